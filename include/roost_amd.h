/*
 * roost_amd.h -- the per-op entry points of the MI355X (gfx950) Roost kernel library, exported by name.
 *
 * A Roost loader reaches these through the registration table that roost_register() fills (RoostOpEntry.run / plan /
 * workspace); they are also exported under the names below so a C, ctypes or P/Invoke caller can bind them directly.
 * Each one replaces the reference entry point named beside it, with the same arguments, statuses and ownership rules
 * (caller-owned workspaces, no allocation, no host synchronisation, typed refusals before any launch).
 */
#ifndef ROOST_AMD_H_
#define ROOST_AMD_H_

#include "roost_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Library identity: the file is libroost_kernels_gfx950.so, roost_register() reports library_name
 * "roost-kernels-gfx950", and every entry's constraints.sm_min is ROOST_AMD_ARCH_ID. */
#define ROOST_AMD_ARCH_ID 950u

/* PagedAttention, variant "paged-attention-gfx950" (DETERMINISTIC | BATCH_INVARIANT | NEEDS_PLAN).
 * Replaces roost_paged_attention_workspace / _plan / _run of the reference
 * (kernels/src/paged_attention.cu:183-198, :200-250, :252-349; declared in kernels/src/roost_internal.h:45-47). */
ROOST_API RoostStatus roost_paged_attention_workspace(RoostContext* ctx, const void* params, RoostWorkspaceSizes* sizes);
ROOST_API RoostStatus roost_paged_attention_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                 void* stream);
ROOST_API RoostStatus roost_paged_attention_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                void* stream);

/* PagedAttention with Qwen3.5's attention output gate (SigmoidMul, out = out * sigmoid(gate)) folded into the kernels
 * that write the output. No counterpart in the reference, whose Qwen3.5 worker runs roost_paged_attention_run and then
 * roost_sigmoid_mul_run on its output (Qwen35EagerModel.cs:94-97 lists both kernels; semantics CpuOps.Gating.cs:84-96).
 * This call computes the same output bit for bit and writes it once: each output element, rounded to the output type,
 * is multiplied by sigmoid(gate) with the SigmoidMul op's own arithmetic where the decode, tile and merge kernels store
 * it. `params` is a planned RoostPagedAttentionParams (plan() and the workspace as for roost_paged_attention_run);
 * `gate_params` a RoostSigmoidMulParams whose input and output are both the attention output (the gate applies in
 * place), rows = tokens, dim = q_heads * head_dim, and whose gate (same dtype as the output, 8-byte aligned) does not
 * overlap the output. The lse output, when requested, is that of the ungated attention. */
ROOST_API RoostStatus roost_amd_paged_attention_gated_run(RoostContext* ctx, const void* params, const void* gate_params,
                                                          const RoostWorkspace* ws, void* stream);

/* CacheWrite, variant "cache-write-gfx950" (GRAPH_CAPTURABLE | DETERMINISTIC | BATCH_INVARIANT), no workspace.
 * Replaces roost_cache_write_run (kernels/src/m0_ops.cu:388-429; declared in kernels/src/roost_internal.h:42). */
ROOST_API RoostStatus roost_cache_write_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                            void* stream);

/* GatedDeltaRule chunked prefill, variant "gated-delta-rule-chunk-gfx950"
 * (DETERMINISTIC | BATCH_INVARIANT | NEEDS_PLAN). Replaces roost_gdn_chunk_workspace / _plan / _run
 * (kernels/src/ops/gated_delta_rule.cu:380-576; declared in kernels/src/roost_internal.h:81-83). */
ROOST_API RoostStatus roost_gdn_chunk_workspace(RoostContext* ctx, const void* params, RoostWorkspaceSizes* sizes);
ROOST_API RoostStatus roost_gdn_chunk_plan(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                           void* stream);
ROOST_API RoostStatus roost_gdn_chunk_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream);

/* GatedDeltaRule recurrent (decode and short continuations), variant "gated-delta-rule-recurrent-aot" -- the id the
 * worker names (reference src/Starlings.Roost.Worker/Eager/CudaOps.cs:28) -- flagged
 * GRAPH_CAPTURABLE | DETERMINISTIC | BATCH_INVARIANT, no plan. Replaces roost_gdn_recurrent_workspace / _run
 * (kernels/src/ops/gated_delta_rule.cu:580-649; declared in kernels/src/roost_internal.h:84-85). */
ROOST_API RoostStatus roost_gdn_recurrent_workspace(RoostContext* ctx, const void* params, RoostWorkspaceSizes* sizes);
ROOST_API RoostStatus roost_gdn_recurrent_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                              void* stream);

/* GatedDeltaRule recurrent variant without a workspace argument. This entry point has no counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). It computes exactly what roost_gdn_recurrent_run computes, with the routing scratch (chunk
 * tables and per-(chunk, head) records of the sequences of 16+ tokens) in a static 24 MiB device array per GPU instead
 * of ws->device. A call whose routing could need more than the array (the workspace query of the recurrent variant
 * reports above 24 MiB: room for 76 chunks of 64 tokens x 16 heads, e.g. one 4,700-token sequence, or a worker step of
 * 1,072 tokens over 50 sequences) is refused with ROOST_STATUS_INVALID_ARGUMENT before any launch. The context's device must be
 * current. Calls that overlap on one GPU race on its array. It calls no hipMalloc/hipFree. */
ROOST_API RoostStatus roost_amd_gdn_recurrent_run_noalloc(RoostContext* ctx, const void* params, void* stream);

/* GatedDeltaRuleGates folded into the recurrent GatedDeltaRule variant. No counterpart in the reference, whose Qwen3.5
 * layer runs roost_gated_delta_rule_gates_run (g, beta from a, b, a_log, dt_bias) and then the recurrent variant on
 * them (CpuOps.Gating.cs:21-58, CpuOps.Hybrid.cs:30-157). This call computes the same outputs and states bit for bit
 * without writing or reading g and beta: each kernel that reads a token's gates computes them from the gates' inputs
 * with the gates op's own arithmetic (beta rounded to bf16, as that op's bf16 output holds it). `params` is a
 * RoostGatedDeltaRuleParams whose g and beta spans are not read; `gates` a RoostGatedDeltaRuleGatesParams (tokens and
 * v_heads equal to the GDN call's; a and b bf16 or f32 row-strided views, a_log and dt_bias bf16 or f32) whose g and
 * beta spans are not read. Workspace as roost_gdn_recurrent_workspace sizes it. */
ROOST_API RoostStatus roost_amd_gdn_recurrent_gated_run(RoostContext* ctx, const void* params, const void* gates,
                                                         const RoostWorkspace* ws, void* stream);

/* One decode step of a Gated DeltaNet layer in one call: CausalConv1d, GatedDeltaRuleGates, the recurrent GatedDeltaRule
 * and GatedRmsNorm. No counterpart in the reference, whose Qwen3.5 worker runs the four ops one after another
 * (Qwen35EagerModel.cs:89-92 lists them; semantics CpuOps.Hybrid.cs:30-157, 160-263 and CpuOps.Gating.cs:21-83). The
 * norm's output, the GDN output, the recurrent states and the convolution states equal the four calls' bit for bit
 * (sequences that share a state slot run in batch order, as the recurrent variant runs them); the convolution's output
 * is not written (its span is only checked). `conv_params` is a RoostCausalConv1dParams
 * over bf16 activations with at most 4 taps and the GDN call's batch, tokens and cu_seqlens; `gdn_params` a
 * RoostGatedDeltaRuleParams whose q, k and v are column views of the convolution's output (row stride = channels) and
 * whose cu_seqlens_host is given: every sequence must be shorter than 16 tokens (longer ones run on the chunk kernels in
 * the recurrent variant), else UNSUPPORTED; `gates_params` a RoostGatedDeltaRuleGatesParams as for
 * roost_amd_gdn_recurrent_gated_run, or NULL to read g and beta from the GDN params; `norm_params` a
 * RoostGatedRmsNormParams of bf16 rows = tokens x v_heads, dim = 128, whose input is the GDN output, with input, gate and
 * output 16-byte aligned, and whose output overlaps none of the layer's other inputs or states. No workspace. */
ROOST_API RoostStatus roost_amd_gdn_decode_layer_run(RoostContext* ctx, const void* conv_params,
                                                      const void* gates_params, const void* gdn_params,
                                                      const void* norm_params, void* stream);

/* One Gated DeltaNet layer of any step (decode, prefill or mixed) over the recurrent variant in one call: CausalConv1d,
 * GatedDeltaRuleGates, GatedDeltaRule and GatedRmsNorm. No counterpart in the reference (the same four calls, one after
 * another; the worker names the recurrent variant for every length, CudaOps.cs:28). A step whose sequences are all
 * shorter than 16 tokens (known from tokens < 16 or from cu_seqlens_host) with the norm in its single-pass bf16 form
 * runs as roost_amd_gdn_decode_layer_run does; any other step runs the convolution, the recurrent variant with g and
 * beta computed from the gates' inputs (its sequences of 16+ tokens on the chunk kernels) and the norm. The norm's
 * output, the recurrent states and the convolution states equal the four calls' bit for bit (the convolution's output
 * is written on the second path only). Params as for roost_amd_gdn_decode_layer_run, without its
 * length limit; `ws` is the recurrent variant's workspace (roost_gdn_recurrent_workspace of `gdn_params`; NULL is
 * enough when it reports zero bytes). */
ROOST_API RoostStatus roost_amd_gdn_layer_run(RoostContext* ctx, const void* conv_params, const void* gates_params,
                                              const void* gdn_params, const void* norm_params, const RoostWorkspace* ws,
                                              void* stream);

/* One prefill pass of a Gated DeltaNet layer over the chunk variant in one call: CausalConv1d, GatedDeltaRuleGates, the
 * chunked GatedDeltaRule and GatedRmsNorm. No counterpart in the reference (the same four calls as above, one after
 * another). The chunk kernels compute g and beta from the gates' inputs where they read them (the gates op's
 * arithmetic), so g and beta never reach memory. The convolution's output, the GDN output, the norm's output, the
 * recurrent states and the convolution states equal the four calls' bit for bit. Params as for
 * roost_amd_gdn_decode_layer_run, except that the sequences may have any lengths (cu_seqlens_host may be NULL at run)
 * and the norm may take any form roost_gated_rms_norm_run takes. `ws` is the chunk variant's workspace, sized by
 * roost_gdn_chunk_workspace and planned by roost_amd_gdn_chunk_layer_plan for the same gates and GDN params (else
 * NOT_PLANNED). */
ROOST_API RoostStatus roost_amd_gdn_chunk_layer_run(RoostContext* ctx, const void* conv_params,
                                                     const void* gates_params, const void* gdn_params,
                                                     const void* norm_params, const RoostWorkspace* ws, void* stream);
/* plan() of roost_amd_gdn_chunk_layer_run: roost_gdn_chunk_plan of `gdn_params` (host chunk tables from cu_seqlens_host,
 * copied to ws on the stream), except that with `gates_params` given the GDN params' g and beta are not read. */
ROOST_API RoostStatus roost_amd_gdn_chunk_layer_plan(RoostContext* ctx, const void* gates_params, const void* gdn_params,
                                                      const RoostWorkspace* ws, void* stream);

/* The Gated DeltaNet layer's neighbour ops, each flagged GRAPH_CAPTURABLE | DETERMINISTIC | BATCH_INVARIANT, no plan
 * and no workspace:
 * GatedDeltaRuleGates, variant "gated-delta-rule-gates-gfx950" -- replaces roost_gated_delta_rule_gates_run
 *   (kernels/src/ops/gating.cu:110-177);
 * GatedRmsNorm, variant "gated-rms-norm-gfx950" -- replaces roost_gated_rms_norm_run (gating.cu:179-229);
 * SigmoidMul, variant "sigmoid-mul-gfx950" -- replaces roost_sigmoid_mul_run (gating.cu:231-269);
 * CausalConv1d, variant "causal-conv1d-gfx950" -- replaces roost_causal_conv1d_run
 *   (kernels/src/ops/causal_conv1d.cu:122-175);
 * RecurrentStateCopy / RecurrentStateSnapshot, variants "recurrent-state-copy-gfx950" / "recurrent-state-snapshot-gfx950"
 *   -- replace roost_recurrent_state_copy_run / _snapshot_run (kernels/src/ops/recurrent_state.cu:58-108).
 * All are registered by kernels/src/ops/hybrid_entries.cu:75-148 in the reference. */
ROOST_API RoostStatus roost_gated_delta_rule_gates_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                       void* stream);
ROOST_API RoostStatus roost_gated_rms_norm_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                               void* stream);
ROOST_API RoostStatus roost_sigmoid_mul_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                            void* stream);
ROOST_API RoostStatus roost_causal_conv1d_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                              void* stream);
ROOST_API RoostStatus roost_recurrent_state_copy_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws,
                                                     void* stream);
ROOST_API RoostStatus roost_recurrent_state_snapshot_run(RoostContext* ctx, const void* params,
                                                         const RoostWorkspace* ws, void* stream);

/* The attention layer's input ops, each flagged GRAPH_CAPTURABLE | DETERMINISTIC | BATCH_INVARIANT, no plan and no
 * workspace:
 * QkNorm, variant "qk-norm-gfx950" -- replaces the reference's QkNormRun (kernels/src/m0_ops.cu:89-130, registered as
 *   "qk-norm-flashinfer" at kernels/src/m0_registry.cu:77);
 * Rope, variant "rope-gfx950" -- replaces RopeRun (kernels/src/m0_ops.cu:210-255, "rope-roost" at m0_registry.cu:79). */
ROOST_API RoostStatus roost_qk_norm_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream);
ROOST_API RoostStatus roost_rope_run(RoostContext* ctx, const void* params, const RoostWorkspace* ws, void* stream);

/* QkvQkNormRopeCacheWrite (ROOST_OP_QKV_QK_NORM_ROPE_CACHE_WRITE, 67), variant "qkv-qk-norm-rope-cache-write-gfx950".
 * The reference's C header names only the op id: the op exists in its CPU reference (src/Starlings.Roost.Ops/
 * CpuOps.Fused.cs:37-95) with the argument struct QkvQkNormRopeCacheWriteArgs (src/Starlings.Roost.Ops/OpArgs.cs:
 * 629-683), and no CUDA library implements it. This record carries those arguments field for field in the ABI's
 * style; the activation type is qkv's dtype and the cache type k_cache's. Each [q | k | v] row of qkv is split: q
 * heads are RmsNormed with q_weight, rotated (full rotary width, default frequencies, NeoX halves) and written to q;
 * k heads are RmsNormed with k_weight, rotated and written into k_cache at slot_mapping[t] (NHD pools, unit scale);
 * v heads are copied into v_cache there. A negative or out-of-pool slot writes no cache row; qkv is left as it was. */
typedef struct RoostQkvQkNormRopeCacheWriteParams {
  uint32_t struct_size;
  uint32_t abi_minor;
  RoostDeviceSpan qkv;          /* [tokens, (q_heads + 2 * kv_heads) * head_dim] */
  RoostDeviceSpan q;            /* [tokens, q_heads, head_dim] output */
  RoostDeviceSpan q_weight;     /* [head_dim] */
  RoostDeviceSpan k_weight;     /* [head_dim] */
  RoostDeviceSpan positions;    /* [tokens] int32 */
  RoostDeviceSpan k_cache;      /* [pages, page_size, kv_heads, head_dim] */
  RoostDeviceSpan v_cache;      /* same */
  RoostDeviceSpan slot_mapping; /* [tokens] int64 */
  uint32_t tokens;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t page_size;
  float eps;
  float theta;
  uint32_t reserved0;
} RoostQkvQkNormRopeCacheWriteParams;

ROOST_API RoostStatus roost_qkv_qk_norm_rope_cache_write_run(RoostContext* ctx, const void* params,
                                                             const RoostWorkspace* ws, void* stream);

/* The plan region: the batch tables and slot mapping of one worker step, from its sequences. Replaces the worker's
 * PlanRegionWriter.Fill (reference src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64), which the reference runs
 * in C# on a host mirror of the region before one host-to-device copy. For sequence b (in order):
 *   q_indptr[b] = cu_seqlens[b] = token_start[b]; kv_indptr[b] = blocks listed before b;
 *   kv_indices[kv_indptr[b] + i] = its block i; kv_last_page_len[b] = kv_length[b] - (its blocks - 1) * block_size;
 *   state_slots[b] = recurrent_slot[b];
 *   for t < token_count[b], at index = token_start[b] + t and position = position_offset[b] + t:
 *     positions[index] = position; slot_mapping[index] = block[position / block_size] * block_size + position % block_size;
 * and the [batch] entries of q_indptr and cu_seqlens are the last sequence's token_start + token_count, of kv_indptr
 * the number of blocks. The region's token ids and sampling rows (embedding and sampler inputs) are not written here.
 * state_slots / recurrent_slot and positions may be NULL (not written). Entries no sequence writes are left alone. */
typedef struct RoostAmdPlanRegion {
  uint32_t batch;                 /* sequences */
  uint32_t tokens;                /* entries of positions and slot_mapping */
  uint32_t block_size;            /* tokens per KV page, > 0 */
  uint32_t reserved0;             /* 0 */
  const int32_t* token_start;     /* [batch] */
  const int32_t* token_count;     /* [batch] */
  const int32_t* position_offset; /* [batch]: position of the sequence's first token of this step */
  const int32_t* kv_length;       /* [batch]: keys after this step */
  const int32_t* block_indptr;    /* [batch + 1], from 0: sequence b's blocks are blocks[block_indptr[b] ..) */
  const int32_t* blocks;          /* [block_indptr[batch]] */
  const int32_t* recurrent_slot;  /* [batch] or NULL */
  int32_t* q_indptr;              /* [batch + 1] */
  int32_t* cu_seqlens;            /* [batch + 1] */
  int32_t* kv_indptr;             /* [batch + 1] */
  int32_t* kv_indices;            /* [block_indptr[batch]] */
  int32_t* kv_last_page_len;      /* [batch] */
  int32_t* state_slots;           /* [batch] or NULL */
  int32_t* positions;             /* [tokens] or NULL */
  int64_t* slot_mapping;          /* [tokens] */
} RoostAmdPlanRegion;

/* Host memory: fills the tables on the calling thread. A sequence whose tokens fall outside [0, tokens), whose
 * positions reach past its blocks, or whose block_indptr goes backwards is refused with ROOST_STATUS_INVALID_ARGUMENT
 * (the reference's Fill throws on the same plans) and nothing is written. */
ROOST_API RoostStatus roost_amd_plan_region_fill(const RoostAmdPlanRegion* region);

/* Device memory: one launch on `stream` writes the same tables on the GPU from the device copies of the sequences'
 * fields, so a step's per-token work never crosses PCIe. The device arrays are not validated on the host: a token
 * index outside [0, tokens) is skipped and a position past its sequence's blocks gets slot -1 (CacheWrite skips it). */
ROOST_API RoostStatus roost_amd_plan_region_run(RoostContext* ctx, const RoostAmdPlanRegion* region, void* stream);

/* The same tables read straight from a C2 step plan: the shared buffer the engine writes (RoostStepPlanHeader and its
 * tables, reference kernels/include/roost_worker_shm.h:57-141), in place of the worker's StepPlanReader.Read +
 * PlanRegionWriter.Fill (src/Starlings.Roost.Worker/Eager/StepPlanReader.cs:195-345, PlanRegionWriter.cs:19-64).
 * Sequence b's KV blocks are the first ceil((position_offset + token_count) / block_size) ids of its group_blocks entry
 * b * group_count + attention_group; its keys after the step are position_offset + token_count. Besides the tables of
 * roost_amd_plan_region_fill it writes ids[index] = token_ids[index] and, for each sequence with the sample flag
 * (0x2) in plan order, rows[r] = its last token index. The plan is checked as the reader checks the fields used here
 * (magic, table bounds and counts, contiguous non-empty token ranges, consecutive positions, group_blocks_start ==
 * b * group_count, enough blocks listed); a plan that fails, or outputs shorter than it needs, is refused with
 * ROOST_STATUS_INVALID_ARGUMENT and nothing is written. Host memory only. */
typedef struct RoostAmdStepTables {
  uint32_t attention_group;  /* the state group whose block lists hold the attention KV blocks */
  uint32_t block_size;       /* tokens per KV page, > 0 */
  uint32_t max_batch;        /* sequences the per-sequence outputs hold (indptr arrays hold max_batch + 1) */
  uint32_t max_tokens;       /* entries of ids, positions and slot_mapping */
  uint32_t max_blocks;       /* entries of kv_indices */
  uint32_t batch;            /* out: sequences */
  uint32_t tokens;           /* out: tokens */
  uint32_t blocks;           /* out: kv_indices entries written */
  uint32_t rows_written;     /* out: sampling rows written */
  uint32_t attention_blocks; /* blocks in the attention KV pool, > 0: block ids outside [0, attention_blocks) are refused */
  int32_t* q_indptr;         /* [batch + 1] */
  int32_t* cu_seqlens;       /* [batch + 1] */
  int32_t* kv_indptr;        /* [batch + 1] */
  int32_t* kv_indices;       /* [blocks] */
  int32_t* kv_last_page_len; /* [batch] */
  int32_t* state_slots;      /* [batch] or NULL */
  int32_t* ids;              /* [tokens] or NULL */
  int32_t* positions;        /* [tokens] or NULL */
  int64_t* slot_mapping;     /* [tokens] */
  int32_t* rows;             /* [max_batch] or NULL */
} RoostAmdStepTables;

ROOST_API RoostStatus roost_amd_plan_region_from_step(const void* plan, uint64_t plan_bytes, RoostAmdStepTables* tables);

#ifdef __cplusplus
}
#endif

#endif /* ROOST_AMD_H_ */
