/*
 * roost_kernels.h -- Roost kernel-library C ABI, major 1 minor 3, as exported by the MI355X (gfx950) HIP library.
 *
 * This header restates the parts of Roost's contract C1 that the attention + Gated DeltaNet library touches:
 * versions, status codes, element types, paged layouts, op ids, registration flags, the shared records
 * (RoostDeviceSpan, RoostWorkspaceSizes, RoostWorkspace, RoostConstraints, RoostContextCreateParams, RoostOpEntry,
 * RoostOpTable), the params of PagedAttention, CacheWrite and GatedDeltaRule, and the five library exports.
 * Every struct layout is byte-identical to the reference header
 * (reference: kernels/include/roost_kernels.h:178-274, :354-381, :465-481, :568-593) so that Roost's C# mirror
 * (Starlings.Roost.Abstractions/Abi/KernelStructs.cs) binds to this library unchanged; the sizes and offsets are
 * asserted against the reference's layout fixture by tests/test_abi.py and by static_asserts in the library.
 *
 * Rules carried over from the contract (reference: kernels/include/roost_kernels.h:10-26):
 *   - fixed-width integers, float, double and pointers only; every params struct starts with struct_size, abi_minor;
 *   - entry points never allocate device memory, never synchronise the host, and treat workspace contents as
 *     undefined on entry (scratch that must start at zero is cleared by the library on the caller's stream);
 *   - errors are returned as a status; roost_last_error() holds the message for the calling thread;
 *   - the stream argument is an opaque pointer: for this library it is a hipStream_t (NULL = the null stream), and
 *     the library links the shared HIP runtime (libamdhip64.so.7) so streams pass between host and library.
 */
#ifndef ROOST_KERNELS_H_
#define ROOST_KERNELS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define ROOST_API __attribute__((visibility("default")))
#else
#define ROOST_API
#endif

/* ---- Versions ---- */
#define ROOST_ABI_MAJOR 1
#define ROOST_ABI_MINOR 3
#define ROOST_ABI_VERSION ((ROOST_ABI_MAJOR << 16) | ROOST_ABI_MINOR) /* what roost_abi_version() returns */

/* ---- Status codes ---- */
typedef int32_t RoostStatus;
#define ROOST_STATUS_OK 0
#define ROOST_STATUS_INVALID_ARGUMENT 1
#define ROOST_STATUS_UNSUPPORTED 2
#define ROOST_STATUS_CUDA_ERROR 3 /* name kept for ABI stability: any GPU runtime error (HIP here) */
#define ROOST_STATUS_INTERNAL 4
#define ROOST_STATUS_ABI_MISMATCH 5
#define ROOST_STATUS_OUT_OF_MEMORY 6
#define ROOST_STATUS_WORKSPACE_TOO_SMALL 7
#define ROOST_STATUS_NOT_PLANNED 8

/* ---- Element types ---- */
#define ROOST_DTYPE_UNDEFINED 0
#define ROOST_DTYPE_F32 1
#define ROOST_DTYPE_F16 2
#define ROOST_DTYPE_BF16 3
#define ROOST_DTYPE_F64 4
#define ROOST_DTYPE_F8E4M3 5
#define ROOST_DTYPE_F8E5M2 6
#define ROOST_DTYPE_I8 7
#define ROOST_DTYPE_U8 8
#define ROOST_DTYPE_I16 9
#define ROOST_DTYPE_I32 10
#define ROOST_DTYPE_U32 11
#define ROOST_DTYPE_I64 12
#define ROOST_DTYPE_U64 13
#define ROOST_DTYPE_I4 14
#define ROOST_DTYPE_U4 15
#define ROOST_DTYPE_F4E2M1 16
#define ROOST_DTYPE_COUNT 17

/* ---- Layouts ---- */
#define ROOST_LAYOUT_ROW_MAJOR 0
#define ROOST_LAYOUT_COL_MAJOR 1
#define ROOST_LAYOUT_PAGED_NHD 2 /* pool [pages, page_size, kv_heads, head_dim] */
#define ROOST_LAYOUT_PAGED_HND 3 /* pool [pages, kv_heads, page_size, head_dim] */

/* ---- Op ids (numbering is permanent; reference kernels/include/roost_kernels.h:106-164) ---- */
#define ROOST_OP_RMS_NORM 1
#define ROOST_OP_QK_NORM 2
#define ROOST_OP_ROPE 3
#define ROOST_OP_PAGED_ATTENTION 4
#define ROOST_OP_SILU_AND_MUL 5
#define ROOST_OP_GELU_AND_MUL 6
#define ROOST_OP_GEMM 7
#define ROOST_OP_EMBEDDING 8
#define ROOST_OP_LM_HEAD 9
#define ROOST_OP_RESIDUAL 10
#define ROOST_OP_CACHE_WRITE 11
#define ROOST_OP_CACHE_COPY 12
#define ROOST_OP_ARGMAX 13
#define ROOST_OP_SAMPLE 14
#define ROOST_OP_ADD_RMS_NORM 64
#define ROOST_OP_ADD_RMS_NORM_QUANT 65
#define ROOST_OP_SILU_MUL_QUANT 66
#define ROOST_OP_QKV_QK_NORM_ROPE_CACHE_WRITE 67
#define ROOST_OP_GEMM_LORA_EPILOGUE 68
#define ROOST_OP_GATED_DELTA_RULE 128
#define ROOST_OP_CAUSAL_CONV1D 129
#define ROOST_OP_RECURRENT_STATE_COPY 130
#define ROOST_OP_RECURRENT_STATE_SNAPSHOT 131
#define ROOST_OP_SLIDING_WINDOW_ATTENTION 132
#define ROOST_OP_GATED_DELTA_RULE_GATES 133
#define ROOST_OP_GATED_RMS_NORM 134
#define ROOST_OP_SIGMOID_MUL 135

/* ---- Registration flags ---- */
#define ROOST_FLAG_GRAPH_CAPTURABLE 0x1u /* run() may be captured in a graph */
#define ROOST_FLAG_DETERMINISTIC 0x2u    /* identical input and launch shape give identical bits */
#define ROOST_FLAG_BATCH_INVARIANT 0x4u  /* a row's result does not depend on the other rows of the call */
#define ROOST_FLAG_NEEDS_PLAN 0x8u       /* plan() runs on the host before run(); plan() is never captured */
#define ROOST_FLAG_PLAN_PER_SHAPE 0x10u  /* one plan serves every call of the same shape bucket */

/* ---- Shared records ---- */

/* A buffer: device address, element count (not bytes) and element type. */
typedef struct RoostDeviceSpan {
  void* address;
  uint64_t length;
  uint32_t dtype; /* ROOST_DTYPE_* */
  uint32_t reserved0;
} RoostDeviceSpan;

/* What an entry's workspace query asks the caller to provide. Zero means none. */
typedef struct RoostWorkspaceSizes {
  uint32_t struct_size;
  uint32_t abi_minor;
  uint64_t device_bytes;
  uint64_t pinned_host_bytes;
  uint64_t plan_bytes;
  uint32_t device_alignment;
  uint32_t reserved0;
} RoostWorkspaceSizes;

/* Caller-owned workspaces, sized from RoostWorkspaceSizes. */
typedef struct RoostWorkspace {
  uint32_t struct_size;
  uint32_t abi_minor;
  void* device;
  uint64_t device_bytes;
  void* pinned_host;
  uint64_t pinned_host_bytes;
  void* plan;
  uint64_t plan_bytes;
} RoostWorkspace;

/* Where a variant is valid. Bit i of head_dim_mask = head_dim 16*(i+1); bit i of page_size_mask = page size 2^i;
 * bit i of group_size_mask = i+1 query heads per KV head. sm_min is the architecture id (950 for gfx950 here). */
typedef struct RoostConstraints {
  uint32_t sm_min;
  uint32_t sm_max;
  uint64_t act_dtype_mask;
  uint64_t weight_dtype_mask;
  uint64_t kv_dtype_mask;
  uint64_t head_dim_mask;
  uint32_t layout_mask;
  uint32_t page_size_mask;
  uint32_t min_alignment;
  uint32_t max_batch;
  uint64_t max_tokens;
  uint32_t group_size_mask;
  uint32_t reserved0;
} RoostConstraints;

typedef struct RoostContext RoostContext;

typedef struct RoostContextCreateParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  int32_t device; /* HIP device ordinal, current on the calling thread */
  uint32_t flags; /* ROOST_CONTEXT_* */
  void* stream;   /* set-up stream; may be NULL */
  uint64_t reserved0;
} RoostContextCreateParams;

#define ROOST_CONTEXT_DETERMINISTIC 0x1u

typedef RoostStatus (*RoostRunFn)(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream);
typedef RoostStatus (*RoostPlanFn)(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream);
typedef RoostStatus (*RoostWorkspaceFn)(RoostContext* ctx, const void* params, RoostWorkspaceSizes* sizes);

typedef struct RoostOpEntry {
  uint32_t op;
  uint32_t flags;
  const char* variant_id;
  uint32_t params_struct_size;
  uint32_t params_abi_minor;
  RoostConstraints constraints;
  RoostRunFn run;
  RoostPlanFn plan;           /* non-NULL exactly when flags has ROOST_FLAG_NEEDS_PLAN */
  RoostWorkspaceFn workspace; /* NULL = no workspace */
  uint64_t reserved0;
} RoostOpEntry;

typedef struct RoostOpTable {
  uint32_t struct_size;  /* caller */
  uint32_t abi_minor;    /* caller */
  uint32_t entry_size;   /* library: sizeof(RoostOpEntry) */
  uint32_t entry_count;  /* library */
  const RoostOpEntry* entries;
  const char* library_name;
  uint32_t library_abi_major;
  uint32_t library_abi_minor;
} RoostOpTable;

/* ---- PagedAttention ---- */
#define ROOST_ATTENTION_DECODE 0
#define ROOST_ATTENTION_PREFILL 1

/* Attention of tokens' queries over a block-tabled KV pool. The *_host pointers are host copies of the batch tables,
 * read only by the workspace query and plan(); run() accepts them NULL. */
typedef struct RoostPagedAttentionParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan q;                /* [tokens, q_heads, head_dim] */
  RoostDeviceSpan output;           /* [tokens, q_heads, head_dim] */
  RoostDeviceSpan lse;              /* optional [tokens, q_heads] f32, base-2 log-sum-exp of the scaled scores */
  RoostDeviceSpan k_cache;          /* pool, layout per kv_layout */
  RoostDeviceSpan v_cache;
  RoostDeviceSpan q_indptr;         /* [batch + 1] i32 */
  RoostDeviceSpan kv_indptr;        /* [batch + 1] i32, offsets into kv_indices */
  RoostDeviceSpan kv_indices;       /* page ids, i32 */
  RoostDeviceSpan kv_last_page_len; /* [batch] i32, 1..page_size */
  const int32_t* q_indptr_host;
  const int32_t* kv_indptr_host;
  const int32_t* kv_last_page_len_host;
  uint32_t mode; /* ROOST_ATTENTION_* */
  uint32_t batch;
  uint32_t tokens;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t kv_layout;
  float sm_scale;        /* 0 = 1/sqrt(head_dim) */
  float logits_soft_cap; /* 0 = off */
  int32_t window_left;   /* -1 = no sliding window */
  uint32_t causal;       /* prefill only */
} RoostPagedAttentionParams;

/* ---- CacheWrite ---- */
/* Token t's K and V rows go to slot slot_mapping[t] = page * page_size + offset; a negative slot skips the token. */
typedef struct RoostCacheWriteParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan k; /* [tokens, kv_heads, head_dim] */
  RoostDeviceSpan v;
  RoostDeviceSpan k_cache;
  RoostDeviceSpan v_cache;
  RoostDeviceSpan slot_mapping; /* [tokens] i64 */
  uint32_t tokens;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t kv_layout;
  float k_scale; /* 1 unless the cache is quantised */
  float v_scale;
  uint32_t reserved0;
} RoostCacheWriteParams;

/* ---- GatedDeltaRule ---- */
/* Per sequence b (tokens cu_seqlens[b]..cu_seqlens[b+1]) and value head h (key head h / (v_heads / k_heads)), with
 * state S[k_dim, v_dim] from slot state_slots[b]: q, k l2-normalised (1/sqrt(sum x^2 + 1e-6)) when l2_norm_qk,
 * q scaled, then per token S = S * exp(g_t); d = beta_t * (v_t - S^T k_t); S = S + k_t d^T; o_t = S^T q_t.
 * q, k, v are row-strided views (stride 0 = contiguous); output, g and beta are contiguous. */
typedef struct RoostGatedDeltaRuleParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan q;           /* [tokens, k_heads, k_dim] at q_stride */
  RoostDeviceSpan k;           /* [tokens, k_heads, k_dim] at k_stride */
  RoostDeviceSpan v;           /* [tokens, v_heads, v_dim] at v_stride */
  RoostDeviceSpan g;           /* [tokens, v_heads] f32 log decay */
  RoostDeviceSpan beta;        /* [tokens, v_heads] */
  RoostDeviceSpan output;      /* [tokens, v_heads, v_dim] */
  RoostDeviceSpan state;       /* pool [slots, v_heads, k_dim, v_dim] f32 */
  RoostDeviceSpan state_slots; /* [batch] i32 */
  RoostDeviceSpan cu_seqlens;  /* [batch + 1] i32 */
  const int32_t* cu_seqlens_host;
  uint32_t batch;
  uint32_t tokens;
  uint32_t k_heads;
  uint32_t v_heads;
  uint32_t k_dim;
  uint32_t v_dim;
  uint32_t q_stride;
  uint32_t k_stride;
  uint32_t v_stride;
  uint32_t use_initial_state;
  uint32_t l2_norm_qk;
  float scale; /* 0 = 1/sqrt(k_dim) */
} RoostGatedDeltaRuleParams;

/* Gates of a Gated DeltaNet layer from its raw a and b projections (ABI 1.2), per token t and value head h:
 * g = -exp(a_log[h]) * softplus(a[t, h] + dt_bias[h]), softplus(x) = log(1 + exp(x)) and x itself above 20;
 * beta = sigmoid(b[t, h]). a and b are row-strided views (0 = v_heads); every span is read or written in its own dtype
 * (Qwen3.5: g f32, beta in the activation type). */
typedef struct RoostGatedDeltaRuleGatesParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan a;       /* [tokens, v_heads] at a_stride */
  RoostDeviceSpan b;       /* [tokens, v_heads] at b_stride */
  RoostDeviceSpan a_log;   /* [v_heads] */
  RoostDeviceSpan dt_bias; /* [v_heads] */
  RoostDeviceSpan g;       /* [tokens, v_heads] output */
  RoostDeviceSpan beta;    /* [tokens, v_heads] output */
  uint32_t tokens;
  uint32_t v_heads;
  uint32_t a_stride;
  uint32_t b_stride;
} RoostGatedDeltaRuleGatesParams;

/* Gated RMS norm, norm before gate (ABI 1.2): out = x * rsqrt(mean(x^2) + eps) * weight * silu(gate) per row of dim;
 * the weight multiplies as stored and has its own dtype. input may alias output. */
typedef struct RoostGatedRmsNormParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan input;  /* [rows, dim] */
  RoostDeviceSpan gate;   /* [rows, dim] */
  RoostDeviceSpan weight; /* [dim] */
  RoostDeviceSpan output; /* [rows, dim] */
  uint32_t rows;
  uint32_t dim;
  float eps;
  uint32_t reserved0;
} RoostGatedRmsNormParams;

/* Per-head RmsNorm of query and key heads, in place (reference kernels/include/roost_kernels.h:307-323). */
typedef struct RoostQkNormParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan q;        /* [tokens, q_heads, head_dim] at q_stride */
  RoostDeviceSpan k;        /* [tokens, kv_heads, head_dim] at k_stride */
  RoostDeviceSpan q_weight; /* [head_dim] */
  RoostDeviceSpan k_weight; /* [head_dim] */
  uint32_t tokens;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t q_stride; /* elements between tokens; 0 means q_heads * head_dim */
  uint32_t k_stride; /* 0 means kv_heads * head_dim */
  float eps;
  uint32_t reserved0;
} RoostQkNormParams;

#define ROOST_ROPE_DEFAULT 0
#define ROOST_ROPE_LLAMA3 1

/* Rotary position embedding of q and k, in place, NeoX (half-split) pairs unless interleaved is set (reference
 * kernels/include/roost_kernels.h:328-347). */
typedef struct RoostRopeParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan q;         /* [tokens, q_heads, head_dim] */
  RoostDeviceSpan k;         /* [tokens, kv_heads, head_dim] */
  RoostDeviceSpan positions; /* [tokens] int32 */
  uint32_t tokens;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t rotary_dim; /* 0 means head_dim */
  uint32_t kind;       /* ROOST_ROPE_* */
  uint32_t interleaved;
  float theta;
  float llama3_factor;
  float llama3_low_freq_factor;
  float llama3_high_freq_factor;
  uint32_t llama3_original_max_position;
} RoostRopeParams;

/* out = input * sigmoid(gate) elementwise over [rows, dim] (ABI 1.2). input may alias output. */
typedef struct RoostSigmoidMulParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan input;  /* [rows, dim] */
  RoostDeviceSpan gate;   /* [rows, dim] */
  RoostDeviceSpan output; /* [rows, dim] */
  uint32_t rows;
  uint32_t dim;
} RoostSigmoidMulParams;

/* Depthwise causal convolution over packed sequences (ABI 1.2): y_t = bias + sum_{j < width} weight[c, j] *
 * x_{t - (width - 1) + j}, the inputs before a sequence's start taken from its slot's conv_state (oldest first), SiLU
 * last when silu is set; afterwards the slot holds the last width - 1 inputs of [state, sequence]. width <= 16. input
 * and output must not overlap; a sequence of zero tokens leaves its slot untouched. */
typedef struct RoostCausalConv1dParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan input;       /* [tokens, channels] */
  RoostDeviceSpan weight;      /* [channels, width] */
  RoostDeviceSpan bias;        /* optional [channels]; NULL address when unused */
  RoostDeviceSpan output;      /* [tokens, channels] */
  RoostDeviceSpan conv_state;  /* pool [slots, channels, width - 1] */
  RoostDeviceSpan state_slots; /* [batch] int32 */
  RoostDeviceSpan cu_seqlens;  /* [batch + 1] int32 */
  uint32_t batch;
  uint32_t tokens;
  uint32_t channels;
  uint32_t width;
  uint32_t silu;
  uint32_t reserved0;
} RoostCausalConv1dParams;

/* Byte copies of slot pairs[i, 0] to slot pairs[i, 1] of pool, slot_bytes each, in pair order (ABI 1.2). */
typedef struct RoostRecurrentStateCopyParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan pool;
  RoostDeviceSpan pairs; /* [count, 2] int32 */
  uint64_t slot_bytes;
  uint32_t count;
  uint32_t reserved0;
} RoostRecurrentStateCopyParams;

/* pairs[i] = (pool slot, snapshot entry); restore == 0 copies slot to snapshot, else snapshot to slot (ABI 1.2). */
typedef struct RoostRecurrentStateSnapshotParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan pool;
  RoostDeviceSpan snapshots;
  RoostDeviceSpan pairs; /* [count, 2] int32 */
  uint64_t slot_bytes;
  uint32_t count;
  uint32_t restore;
} RoostRecurrentStateSnapshotParams;

/* ---- Exports (reference kernels/include/roost_kernels.h:699-711) ---- */
ROOST_API uint32_t roost_abi_version(void);
ROOST_API const char* roost_last_error(void); /* never NULL; valid until the next call on this thread */
ROOST_API RoostStatus roost_register(RoostOpTable* table);
ROOST_API RoostStatus roost_context_create(const RoostContextCreateParams* params, RoostContext** out);
ROOST_API RoostStatus roost_context_destroy(RoostContext* ctx);

typedef uint32_t (*RoostAbiVersionFn)(void);
typedef const char* (*RoostLastErrorFn)(void);
typedef RoostStatus (*RoostRegisterFn)(RoostOpTable* table);
typedef RoostStatus (*RoostContextCreateFn)(const RoostContextCreateParams* params, RoostContext** out);
typedef RoostStatus (*RoostContextDestroyFn)(RoostContext* ctx);

#ifdef __cplusplus
}
#endif

#endif /* ROOST_KERNELS_H_ */
