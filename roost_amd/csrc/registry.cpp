// The five C1 exports and the registration table of the gfx950 Roost kernel library.
//
// Behaviour follows the reference's registry (kernels/src/registry.cu:60-143): a thread-local last-error string that is
// never NULL, roost_register() filling a caller-owned RoostOpTable with static entries that live until unload, and
// roost_context_create()/destroy() managing a per-device context. Unlike the reference there is no cuBLASLt handle and
// no module loading: every kernel is compiled into this library for gfx950, so a context only records its device.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstring>
#include <new>
#include <string>

#include "common.h"

// The ABI layouts must match the reference header byte for byte (fixture: abi-layout.golden.txt of the reference's
// Starlings.Roost.Abstractions.Tests). A mismatch fails the build here rather than corrupting a caller's struct.
static_assert(sizeof(RoostDeviceSpan) == 24 && offsetof(RoostDeviceSpan, dtype) == 16, "RoostDeviceSpan layout");
static_assert(sizeof(RoostWorkspaceSizes) == 40 && offsetof(RoostWorkspaceSizes, device_alignment) == 32, "sizes");
static_assert(sizeof(RoostWorkspace) == 56 && offsetof(RoostWorkspace, plan_bytes) == 48, "RoostWorkspace layout");
static_assert(sizeof(RoostConstraints) == 72 && offsetof(RoostConstraints, group_size_mask) == 64, "constraints");
static_assert(sizeof(RoostContextCreateParams) == 32 && offsetof(RoostContextCreateParams, stream) == 16, "ctx");
static_assert(sizeof(RoostOpEntry) == 128 && offsetof(RoostOpEntry, run) == 96 && offsetof(RoostOpEntry, workspace) == 112,
              "RoostOpEntry layout");
static_assert(sizeof(RoostOpTable) == 40 && offsetof(RoostOpTable, library_name) == 24, "RoostOpTable layout");
static_assert(sizeof(RoostPagedAttentionParams) == 296 && offsetof(RoostPagedAttentionParams, q_indptr_host) == 224 &&
                  offsetof(RoostPagedAttentionParams, mode) == 248 && offsetof(RoostPagedAttentionParams, causal) == 292,
              "RoostPagedAttentionParams layout");
static_assert(sizeof(RoostCacheWriteParams) == 160 && offsetof(RoostCacheWriteParams, slot_mapping) == 104 &&
                  offsetof(RoostCacheWriteParams, v_scale) == 152,
              "RoostCacheWriteParams layout");
static_assert(sizeof(RoostGatedDeltaRuleParams) == 280 && offsetof(RoostGatedDeltaRuleParams, cu_seqlens_host) == 224 &&
                  offsetof(RoostGatedDeltaRuleParams, use_initial_state) == 268 &&
                  offsetof(RoostGatedDeltaRuleParams, scale) == 276,
              "RoostGatedDeltaRuleParams layout");

static_assert(sizeof(RoostGatedDeltaRuleGatesParams) == 168 && offsetof(RoostGatedDeltaRuleGatesParams, tokens) == 152,
              "RoostGatedDeltaRuleGatesParams layout");
static_assert(sizeof(RoostGatedRmsNormParams) == 120 && offsetof(RoostGatedRmsNormParams, eps) == 112,
              "RoostGatedRmsNormParams layout");
static_assert(sizeof(RoostSigmoidMulParams) == 88 && offsetof(RoostSigmoidMulParams, rows) == 80, "RoostSigmoidMulParams layout");
static_assert(sizeof(RoostCausalConv1dParams) == 200 && offsetof(RoostCausalConv1dParams, batch) == 176 &&
                  offsetof(RoostCausalConv1dParams, silu) == 192,
              "RoostCausalConv1dParams layout");
static_assert(sizeof(RoostQkNormParams) == 136 && offsetof(RoostQkNormParams, tokens) == 104 &&
                  offsetof(RoostQkNormParams, eps) == 128, "RoostQkNormParams layout");
static_assert(sizeof(RoostRopeParams) == 128 && offsetof(RoostRopeParams, tokens) == 80 &&
                  offsetof(RoostRopeParams, theta) == 108 && offsetof(RoostRopeParams, llama3_original_max_position) == 124,
              "RoostRopeParams layout");
static_assert(sizeof(RoostQkvQkNormRopeCacheWriteParams) == 232 &&
                  offsetof(RoostQkvQkNormRopeCacheWriteParams, slot_mapping) == 176 &&
                  offsetof(RoostQkvQkNormRopeCacheWriteParams, tokens) == 200 &&
                  offsetof(RoostQkvQkNormRopeCacheWriteParams, theta) == 224,
              "RoostQkvQkNormRopeCacheWriteParams layout");
static_assert(sizeof(RoostRecurrentStateCopyParams) == 72 && offsetof(RoostRecurrentStateCopyParams, slot_bytes) == 56,
              "RoostRecurrentStateCopyParams layout");
static_assert(sizeof(RoostRecurrentStateSnapshotParams) == 96 &&
                  offsetof(RoostRecurrentStateSnapshotParams, restore) == 92,
              "RoostRecurrentStateSnapshotParams layout");

namespace {

thread_local std::string g_last_error;

using roost::DtypeMask;

constexpr uint64_t HeadDimBit(uint32_t d) { return uint64_t{1} << (d / 16 - 1); }
constexpr uint32_t kPaged = (1u << ROOST_LAYOUT_PAGED_NHD) | (1u << ROOST_LAYOUT_PAGED_HND);
constexpr uint32_t kAnyPageSize = 0xFFu;  // bit i = page size 2^i: 1 .. 128 tokens
constexpr uint32_t kGroup4 = 1u << 3;     // 4 query heads per KV head (bit g - 1: group size g)
constexpr uint32_t kGroups = kGroup4 | (1u << 7) | (1u << 15) | (1u << 31);  // 4, 8, 16 and 32

RoostConstraints BaseConstraints() {
  RoostConstraints c{};
  c.sm_min = ROOST_AMD_ARCH_ID;
  return c;
}

RoostConstraints AttentionConstraints() {
  RoostConstraints c = BaseConstraints();
  c.act_dtype_mask = DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F32);
  c.kv_dtype_mask = DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F32);
  c.head_dim_mask = HeadDimBit(64) | HeadDimBit(128) | HeadDimBit(256);
  c.layout_mask = kPaged;
  c.page_size_mask = kAnyPageSize;
  c.min_alignment = 16;
  c.group_size_mask = kGroups;
  return c;
}

RoostConstraints CacheWriteConstraints() {
  RoostConstraints c = BaseConstraints();
  c.act_dtype_mask = DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F16) | DtypeMask(ROOST_DTYPE_F32);
  c.kv_dtype_mask = c.act_dtype_mask;
  c.head_dim_mask = ~uint64_t{0};
  c.layout_mask = kPaged;
  c.page_size_mask = kAnyPageSize;
  c.min_alignment = 2;
  return c;
}

RoostConstraints GdnConstraints() {
  RoostConstraints c = BaseConstraints();
  c.act_dtype_mask = DtypeMask(ROOST_DTYPE_BF16);
  c.head_dim_mask = HeadDimBit(128);
  c.layout_mask = 1u << ROOST_LAYOUT_ROW_MAJOR;
  c.min_alignment = 16;
  c.group_size_mask = 0xFFu;  // 1 to 8 value heads per key head
  return c;
}

// The GDN layer's elementwise and row ops: bf16 or f32 activations, row-major, element alignment.
RoostConstraints PlainConstraints(uint64_t act_mask, uint32_t alignment) {
  RoostConstraints c = BaseConstraints();
  c.act_dtype_mask = act_mask;
  c.layout_mask = 1u << ROOST_LAYOUT_ROW_MAJOR;
  c.min_alignment = alignment;
  return c;
}

// QkNorm and Rope: bf16 or f32 heads of any even width up to 1024, element alignment (16-byte rows take vector loads).
RoostConstraints HeadConstraints() {
  RoostConstraints c = PlainConstraints(DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F32), 2);
  c.head_dim_mask = ~uint64_t{0};
  return c;
}

// The fused QKV op writes NHD pages of the activation type, or f32 pages under bf16 activations.
RoostConstraints QkvConstraints() {
  RoostConstraints c = HeadConstraints();
  c.kv_dtype_mask = DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F32);
  c.layout_mask = 1u << ROOST_LAYOUT_PAGED_NHD;
  c.page_size_mask = kAnyPageSize;
  return c;
}

RoostOpEntry Entry(uint32_t op, uint32_t flags, const char* id, uint32_t params_size, const RoostConstraints& c,
                   RoostRunFn run, RoostPlanFn plan, RoostWorkspaceFn workspace) {
  RoostOpEntry e{};
  e.op = op;
  e.flags = flags;
  e.variant_id = id;
  e.params_struct_size = params_size;
  e.params_abi_minor = ROOST_ABI_MINOR;
  e.constraints = c;
  e.run = run;
  e.plan = plan;
  e.workspace = workspace;
  return e;
}

constexpr uint32_t kDet = ROOST_FLAG_DETERMINISTIC | ROOST_FLAG_BATCH_INVARIANT;
constexpr uint64_t kBf16F32 = DtypeMask(ROOST_DTYPE_BF16) | DtypeMask(ROOST_DTYPE_F32);

const RoostOpEntry* Entries(uint32_t* count) {
  static const RoostOpEntry entries[] = {
      Entry(ROOST_OP_PAGED_ATTENTION, ROOST_FLAG_DETERMINISTIC | ROOST_FLAG_NEEDS_PLAN, "paged-attention-gfx950",
            sizeof(RoostPagedAttentionParams), AttentionConstraints(), roost_paged_attention_run,
            roost_paged_attention_plan, roost_paged_attention_workspace),
      Entry(ROOST_OP_CACHE_WRITE, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "cache-write-gfx950", sizeof(RoostCacheWriteParams),
            CacheWriteConstraints(), roost_cache_write_run, nullptr, nullptr),
      Entry(ROOST_OP_GATED_DELTA_RULE, kDet | ROOST_FLAG_NEEDS_PLAN, "gated-delta-rule-chunk-gfx950",
            sizeof(RoostGatedDeltaRuleParams), GdnConstraints(), roost_gdn_chunk_run, roost_gdn_chunk_plan,
            roost_gdn_chunk_workspace),
      Entry(ROOST_OP_GATED_DELTA_RULE, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "gated-delta-rule-recurrent-aot",
            sizeof(RoostGatedDeltaRuleParams), GdnConstraints(), roost_gdn_recurrent_run, nullptr,
            roost_gdn_recurrent_workspace),
      Entry(ROOST_OP_CAUSAL_CONV1D, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "causal-conv1d-gfx950",
            sizeof(RoostCausalConv1dParams), PlainConstraints(kBf16F32, 4), roost_causal_conv1d_run, nullptr, nullptr),
      Entry(ROOST_OP_RECURRENT_STATE_COPY, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "recurrent-state-copy-gfx950",
            sizeof(RoostRecurrentStateCopyParams), PlainConstraints(0, 1), roost_recurrent_state_copy_run, nullptr,
            nullptr),
      Entry(ROOST_OP_RECURRENT_STATE_SNAPSHOT, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "recurrent-state-snapshot-gfx950",
            sizeof(RoostRecurrentStateSnapshotParams), PlainConstraints(0, 1), roost_recurrent_state_snapshot_run,
            nullptr, nullptr),
      Entry(ROOST_OP_GATED_DELTA_RULE_GATES, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "gated-delta-rule-gates-gfx950",
            sizeof(RoostGatedDeltaRuleGatesParams), PlainConstraints(kBf16F32, 4), roost_gated_delta_rule_gates_run,
            nullptr, nullptr),
      Entry(ROOST_OP_GATED_RMS_NORM, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "gated-rms-norm-gfx950",
            sizeof(RoostGatedRmsNormParams), PlainConstraints(kBf16F32, 4), roost_gated_rms_norm_run, nullptr, nullptr),
      Entry(ROOST_OP_SIGMOID_MUL, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "sigmoid-mul-gfx950", sizeof(RoostSigmoidMulParams),
            PlainConstraints(kBf16F32, 4), roost_sigmoid_mul_run, nullptr, nullptr),
      Entry(ROOST_OP_QK_NORM, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "qk-norm-gfx950", sizeof(RoostQkNormParams),
            HeadConstraints(), roost_qk_norm_run, nullptr, nullptr),
      Entry(ROOST_OP_ROPE, kDet | ROOST_FLAG_GRAPH_CAPTURABLE, "rope-gfx950", sizeof(RoostRopeParams), HeadConstraints(),
            roost_rope_run, nullptr, nullptr),
      Entry(ROOST_OP_QKV_QK_NORM_ROPE_CACHE_WRITE, kDet | ROOST_FLAG_GRAPH_CAPTURABLE,
            "qkv-qk-norm-rope-cache-write-gfx950", sizeof(RoostQkvQkNormRopeCacheWriteParams), QkvConstraints(),
            roost_qkv_qk_norm_rope_cache_write_run, nullptr, nullptr),
  };
  *count = static_cast<uint32_t>(sizeof(entries) / sizeof(entries[0]));
  return entries;
}

}  // namespace

void roost_set_error(const char* message) { g_last_error = message != nullptr ? message : ""; }

extern "C" {

ROOST_API uint32_t roost_abi_version(void) { return ROOST_ABI_VERSION; }

ROOST_API const char* roost_last_error(void) { return g_last_error.c_str(); }

ROOST_API RoostStatus roost_register(RoostOpTable* table) {
  roost::Gate gate("register");
  gate.Expect(table != nullptr, ROOST_STATUS_INVALID_ARGUMENT, "no op table to fill was passed");
  ROOST_GATE_RETURN(gate);
  gate.Expect(table->struct_size >= sizeof(RoostOpTable) && table->abi_minor <= ROOST_ABI_MINOR,
              ROOST_STATUS_ABI_MISMATCH, "op table of %u bytes at ABI minor %u; this library fills %zu bytes at minor <= %u",
              table->struct_size, table->abi_minor, sizeof(RoostOpTable), static_cast<uint32_t>(ROOST_ABI_MINOR));
  ROOST_GATE_RETURN(gate);
  uint32_t count = 0;
  const RoostOpEntry* entries = Entries(&count);
  table->entry_size = static_cast<uint32_t>(sizeof(RoostOpEntry));
  table->entry_count = count;
  table->entries = entries;
  table->library_name = "roost-kernels-gfx950";
  table->library_abi_major = ROOST_ABI_MAJOR;
  table->library_abi_minor = ROOST_ABI_MINOR;
  return ROOST_STATUS_OK;
}

}  // extern "C"


extern "C" {

ROOST_API RoostStatus roost_context_create(const RoostContextCreateParams* params, RoostContext** out) {
  roost::Gate gate("context_create");
  gate.Expect(params != nullptr && out != nullptr, ROOST_STATUS_INVALID_ARGUMENT,
              "both the create params and the out-pointer are required");
  ROOST_GATE_RETURN(gate);
  gate.Header(params, sizeof(RoostContextCreateParams))
      .Expect(params->reserved0 == 0, ROOST_STATUS_INVALID_ARGUMENT, "reserved0 = %llu, must be 0", static_cast<unsigned long long>(params->reserved0));
  ROOST_GATE_RETURN(gate);
  // The compute-unit count sizes the decode grid; without a visible device (CPU-only validation) 256 is assumed.
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, params->device) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  *out = new (std::nothrow) RoostContext{params->device, params->flags, static_cast<uint32_t>(cus)};
  gate.Expect(*out != nullptr, ROOST_STATUS_OUT_OF_MEMORY, "no host memory left for a context");
  return gate.status();
}

ROOST_API RoostStatus roost_context_destroy(RoostContext* ctx) {
  delete ctx;
  return ROOST_STATUS_OK;
}

}  // extern "C"
