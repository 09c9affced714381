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

#ifdef __cplusplus
}
#endif

#endif /* ROOST_AMD_H_ */
