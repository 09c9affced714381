"""ctypes mirror of the C ABI in include/roost_kernels.h (Roost contract C1, ABI 1.3).

Field order and types follow the header exactly; tests/test_abi.py checks every size and offset against the reference
layout fixture (tests/golden/abi_layout.golden.txt, taken from the reference's
tests/Starlings.Roost.Abstractions.Tests/Layout/abi-layout.golden.txt).
"""
from __future__ import annotations

import ctypes as C

ABI_MAJOR, ABI_MINOR = 1, 3
ABI_VERSION = (ABI_MAJOR << 16) | ABI_MINOR

# Status codes
OK, INVALID_ARGUMENT, UNSUPPORTED, GPU_ERROR, INTERNAL, ABI_MISMATCH, OUT_OF_MEMORY, WORKSPACE_TOO_SMALL, \
    NOT_PLANNED = range(9)
STATUS_NAMES = ["OK", "INVALID_ARGUMENT", "UNSUPPORTED", "CUDA_ERROR", "INTERNAL", "ABI_MISMATCH", "OUT_OF_MEMORY",
                "WORKSPACE_TOO_SMALL", "NOT_PLANNED"]

# Element types
DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_F64 = 1, 2, 3, 4
DTYPE_U8, DTYPE_I32, DTYPE_I64 = 8, 10, 12

# Layouts
LAYOUT_ROW_MAJOR, LAYOUT_PAGED_NHD, LAYOUT_PAGED_HND = 0, 2, 3

# Op ids
OP_PAGED_ATTENTION, OP_CACHE_WRITE, OP_GATED_DELTA_RULE = 4, 11, 128
OP_CAUSAL_CONV1D, OP_RECURRENT_STATE_COPY, OP_RECURRENT_STATE_SNAPSHOT = 129, 130, 131
OP_GATED_DELTA_RULE_GATES, OP_GATED_RMS_NORM, OP_SIGMOID_MUL = 133, 134, 135
OP_QK_NORM, OP_ROPE, OP_QKV_QK_NORM_ROPE_CACHE_WRITE = 2, 3, 67
ROPE_DEFAULT, ROPE_LLAMA3 = 0, 1

# Flags
FLAG_GRAPH_CAPTURABLE, FLAG_DETERMINISTIC, FLAG_BATCH_INVARIANT, FLAG_NEEDS_PLAN, FLAG_PLAN_PER_SHAPE = \
    0x1, 0x2, 0x4, 0x8, 0x10

ATTENTION_DECODE, ATTENTION_PREFILL = 0, 1


class DeviceSpan(C.Structure):
    _fields_ = [("address", C.c_void_p), ("length", C.c_uint64), ("dtype", C.c_uint32), ("reserved0", C.c_uint32)]


class WorkspaceSizes(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("device_bytes", C.c_uint64),
                ("pinned_host_bytes", C.c_uint64), ("plan_bytes", C.c_uint64), ("device_alignment", C.c_uint32),
                ("reserved0", C.c_uint32)]


class Workspace(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("device", C.c_void_p),
                ("device_bytes", C.c_uint64), ("pinned_host", C.c_void_p), ("pinned_host_bytes", C.c_uint64),
                ("plan", C.c_void_p), ("plan_bytes", C.c_uint64)]


class Constraints(C.Structure):
    _fields_ = [("sm_min", C.c_uint32), ("sm_max", C.c_uint32), ("act_dtype_mask", C.c_uint64),
                ("weight_dtype_mask", C.c_uint64), ("kv_dtype_mask", C.c_uint64), ("head_dim_mask", C.c_uint64),
                ("layout_mask", C.c_uint32), ("page_size_mask", C.c_uint32), ("min_alignment", C.c_uint32),
                ("max_batch", C.c_uint32), ("max_tokens", C.c_uint64), ("group_size_mask", C.c_uint32),
                ("reserved0", C.c_uint32)]


class ContextCreateParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("device", C.c_int32), ("flags", C.c_uint32),
                ("stream", C.c_void_p), ("reserved0", C.c_uint64)]


RunFn = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p)
PlanFn = RunFn
WorkspaceFn = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p)


class OpEntry(C.Structure):
    _fields_ = [("op", C.c_uint32), ("flags", C.c_uint32), ("variant_id", C.c_char_p),
                ("params_struct_size", C.c_uint32), ("params_abi_minor", C.c_uint32), ("constraints", Constraints),
                ("run", C.c_void_p), ("plan", C.c_void_p), ("workspace", C.c_void_p), ("reserved0", C.c_uint64)]


class OpTable(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("entry_size", C.c_uint32),
                ("entry_count", C.c_uint32), ("entries", C.c_void_p), ("library_name", C.c_char_p),
                ("library_abi_major", C.c_uint32), ("library_abi_minor", C.c_uint32)]


class PagedAttentionParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("q", DeviceSpan), ("output", DeviceSpan),
                ("lse", DeviceSpan), ("k_cache", DeviceSpan), ("v_cache", DeviceSpan), ("q_indptr", DeviceSpan),
                ("kv_indptr", DeviceSpan), ("kv_indices", DeviceSpan), ("kv_last_page_len", DeviceSpan),
                ("q_indptr_host", C.c_void_p), ("kv_indptr_host", C.c_void_p), ("kv_last_page_len_host", C.c_void_p),
                ("mode", C.c_uint32), ("batch", C.c_uint32), ("tokens", C.c_uint32), ("q_heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("page_size", C.c_uint32),
                ("kv_layout", C.c_uint32), ("sm_scale", C.c_float), ("logits_soft_cap", C.c_float),
                ("window_left", C.c_int32), ("causal", C.c_uint32)]


class CacheWriteParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("k", DeviceSpan), ("v", DeviceSpan),
                ("k_cache", DeviceSpan), ("v_cache", DeviceSpan), ("slot_mapping", DeviceSpan),
                ("tokens", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("page_size", C.c_uint32), ("kv_layout", C.c_uint32), ("k_scale", C.c_float),
                ("v_scale", C.c_float), ("reserved0", C.c_uint32)]


class GatedDeltaRuleParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("q", DeviceSpan), ("k", DeviceSpan),
                ("v", DeviceSpan), ("g", DeviceSpan), ("beta", DeviceSpan), ("output", DeviceSpan),
                ("state", DeviceSpan), ("state_slots", DeviceSpan), ("cu_seqlens", DeviceSpan),
                ("cu_seqlens_host", C.c_void_p), ("batch", C.c_uint32), ("tokens", C.c_uint32),
                ("k_heads", C.c_uint32), ("v_heads", C.c_uint32), ("k_dim", C.c_uint32), ("v_dim", C.c_uint32),
                ("q_stride", C.c_uint32), ("k_stride", C.c_uint32), ("v_stride", C.c_uint32),
                ("use_initial_state", C.c_uint32), ("l2_norm_qk", C.c_uint32), ("scale", C.c_float)]


class GatedDeltaRuleGatesParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("a", DeviceSpan), ("b", DeviceSpan),
                ("a_log", DeviceSpan), ("dt_bias", DeviceSpan), ("g", DeviceSpan), ("beta", DeviceSpan),
                ("tokens", C.c_uint32), ("v_heads", C.c_uint32), ("a_stride", C.c_uint32), ("b_stride", C.c_uint32)]


class GatedRmsNormParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("input", DeviceSpan), ("gate", DeviceSpan),
                ("weight", DeviceSpan), ("output", DeviceSpan), ("rows", C.c_uint32), ("dim", C.c_uint32),
                ("eps", C.c_float), ("reserved0", C.c_uint32)]


class QkNormParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("q", DeviceSpan), ("k", DeviceSpan),
                ("q_weight", DeviceSpan), ("k_weight", DeviceSpan), ("tokens", C.c_uint32), ("q_heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("q_stride", C.c_uint32), ("k_stride", C.c_uint32),
                ("eps", C.c_float), ("reserved0", C.c_uint32)]


class RopeParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("q", DeviceSpan), ("k", DeviceSpan),
                ("positions", DeviceSpan), ("tokens", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32), ("kind", C.c_uint32),
                ("interleaved", C.c_uint32), ("theta", C.c_float), ("llama3_factor", C.c_float),
                ("llama3_low_freq_factor", C.c_float), ("llama3_high_freq_factor", C.c_float),
                ("llama3_original_max_position", C.c_uint32)]


class QkvQkNormRopeCacheWriteParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("qkv", DeviceSpan), ("q", DeviceSpan),
                ("q_weight", DeviceSpan), ("k_weight", DeviceSpan), ("positions", DeviceSpan), ("k_cache", DeviceSpan),
                ("v_cache", DeviceSpan), ("slot_mapping", DeviceSpan), ("tokens", C.c_uint32),
                ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("page_size", C.c_uint32), ("eps", C.c_float), ("theta", C.c_float), ("reserved0", C.c_uint32)]


class SigmoidMulParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("input", DeviceSpan), ("gate", DeviceSpan),
                ("output", DeviceSpan), ("rows", C.c_uint32), ("dim", C.c_uint32)]


class CausalConv1dParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("input", DeviceSpan), ("weight", DeviceSpan),
                ("bias", DeviceSpan), ("output", DeviceSpan), ("conv_state", DeviceSpan), ("state_slots", DeviceSpan),
                ("cu_seqlens", DeviceSpan), ("batch", C.c_uint32), ("tokens", C.c_uint32), ("channels", C.c_uint32),
                ("width", C.c_uint32), ("silu", C.c_uint32), ("reserved0", C.c_uint32)]


class RecurrentStateCopyParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("pool", DeviceSpan), ("pairs", DeviceSpan),
                ("slot_bytes", C.c_uint64), ("count", C.c_uint32), ("reserved0", C.c_uint32)]


class RecurrentStateSnapshotParams(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_minor", C.c_uint32), ("pool", DeviceSpan), ("snapshots", DeviceSpan),
                ("pairs", DeviceSpan), ("slot_bytes", C.c_uint64), ("count", C.c_uint32), ("restore", C.c_uint32)]


class PlanRegion(C.Structure):
    """RoostAmdPlanRegion: plain pointers (host memory for roost_amd_plan_region_fill, device memory for _run)."""
    _fields_ = [("batch", C.c_uint32), ("tokens", C.c_uint32), ("block_size", C.c_uint32), ("reserved0", C.c_uint32)] + [
        (name, C.c_void_p) for name in ("token_start", "token_count", "position_offset", "kv_length", "block_indptr",
                                        "blocks", "recurrent_slot", "q_indptr", "cu_seqlens", "kv_indptr", "kv_indices",
                                        "kv_last_page_len", "state_slots", "positions", "slot_mapping")]


class StepTables(C.Structure):
    """RoostAmdStepTables: the outputs of roost_amd_plan_region_from_step (host pointers)."""
    _fields_ = [(name, C.c_uint32) for name in ("attention_group", "block_size", "max_batch", "max_tokens", "max_blocks",
                                                "batch", "tokens", "blocks", "rows_written", "attention_blocks")] + [
        (name, C.c_void_p) for name in ("q_indptr", "cu_seqlens", "kv_indptr", "kv_indices", "kv_last_page_len",
                                        "state_slots", "ids", "positions", "slot_mapping", "rows")]


# ---- The C2 step plan (reference kernels/include/roost_worker_shm.h:41-141), for building plan buffers ------------------

class TableRef(C.Structure):
    _fields_ = [("offset", C.c_uint64), ("count", C.c_uint32), ("stride", C.c_uint32)]


class StepPlanHeader(C.Structure):
    _fields_ = ([(n, C.c_uint32) for n in ("magic", "layout_version", "header_size", "flags")]
                + [("step_id", C.c_uint64), ("total_bytes", C.c_uint64)]
                + [(n, C.c_uint32) for n in ("shape_bucket", "math_mode", "sequence_count", "token_count", "group_count",
                                             "rank", "mesh_id", "reserved0")]
                + [(n, TableRef) for n in ("sequences", "token_ids", "positions", "group_blocks", "block_ids", "sampling",
                                           "cache_ops", "embedding_inputs", "stop_token_ids", "spec_tree_parents",
                                           "spec_tree_masks", "moe_expert_counts", "moe_expert_placement",
                                           "kv_transfers", "head_rows", "encoder_outputs")]
                + [(n, C.c_uint64) for n in ("reserved1", "reserved2", "input_step_id")])


class PlanSequence(C.Structure):
    _fields_ = ([("sequence_handle", C.c_uint64)]
                + [(n, C.c_uint32) for n in ("token_start", "token_count", "position_offset", "group_blocks_start")]
                + [(n, C.c_int32) for n in ("recurrent_slot", "lora_slot", "grammar_slot", "embedding_slot")]
                + [(n, C.c_uint32) for n in ("sampling_index", "draft_count", "flags", "stop_start", "stop_count",
                                             "max_new_tokens_left", "spec_tree_start", "spec_tree_count")]
                + [(n, C.c_int32) for n in ("head_row", "encoder_output")])


class PlanGroupBlocks(C.Structure):
    _fields_ = [("block_start", C.c_uint32), ("block_count", C.c_uint32)]


SHM_STRUCTS = {"RoostTableRef": TableRef, "RoostStepPlanHeader": StepPlanHeader, "RoostPlanSequence": PlanSequence,
               "RoostPlanGroupBlocks": PlanGroupBlocks}
SHM_MAGIC_PLAN = 0x4C505352  # "RSPL"
SHM_LAYOUT_VERSION = 3
SEQ_FLAG_PREFILL, SEQ_FLAG_SAMPLE = 0x1, 0x2


ALL_STRUCTS = {
    "RoostDeviceSpan": DeviceSpan, "RoostWorkspaceSizes": WorkspaceSizes, "RoostWorkspace": Workspace,
    "RoostConstraints": Constraints, "RoostContextCreateParams": ContextCreateParams, "RoostOpEntry": OpEntry,
    "RoostOpTable": OpTable, "RoostPagedAttentionParams": PagedAttentionParams,
    "RoostCacheWriteParams": CacheWriteParams, "RoostGatedDeltaRuleParams": GatedDeltaRuleParams,
    "RoostGatedDeltaRuleGatesParams": GatedDeltaRuleGatesParams, "RoostGatedRmsNormParams": GatedRmsNormParams,
    "RoostSigmoidMulParams": SigmoidMulParams, "RoostCausalConv1dParams": CausalConv1dParams,
    "RoostRecurrentStateCopyParams": RecurrentStateCopyParams,
    "RoostRecurrentStateSnapshotParams": RecurrentStateSnapshotParams, "RoostQkNormParams": QkNormParams,
    "RoostRopeParams": RopeParams,
}

# Records of this library with no counterpart in the reference's C header (so not in its layout fixture).
EXTENSION_STRUCTS = {"RoostQkvQkNormRopeCacheWriteParams": QkvQkNormRopeCacheWriteParams}


def new(struct_type):
    """A zeroed params/record struct with struct_size and abi_minor filled in."""
    s = struct_type()
    s.struct_size = C.sizeof(struct_type)
    s.abi_minor = ABI_MINOR
    return s
