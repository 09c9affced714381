"""The drop-in boundary without a GPU: struct layouts against the reference's layout fixture, the exported symbols,
the registration table, and the typed refusals that happen before any launch."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

import roost_amd
from roost_amd import abi

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = Path(__file__).resolve().parent / "golden" / "abi_layout.golden.txt"


def parse_golden():
    structs, cur = {}, None
    for line in GOLDEN.read_text().splitlines():
        if line.startswith("#") or not line.strip():
            continue
        m = re.match(r"struct (\w+) size=(\d+) align=(\d+)", line)
        if m:
            cur = m.group(1)
            structs[cur] = {"size": int(m.group(2)), "fields": []}
            continue
        name, off, size, _type = line.split()
        structs[cur]["fields"].append((name, int(off), int(size)))
    return structs


def test_layouts_match_reference_fixture():
    golden = parse_golden()
    assert set(golden) == set(abi.ALL_STRUCTS)
    for name, st in abi.ALL_STRUCTS.items():
        g = golden[name]
        assert C.sizeof(st) == g["size"], name
        fields = [(f[0], getattr(st, f[0]).offset, getattr(st, f[0]).size) for f in st._fields_]
        assert fields == g["fields"], name


def test_extension_layouts_match_the_header():
    """RoostQkvQkNormRopeCacheWriteParams has no reference layout: its ctypes mirror must match the C header's
    offsets, which registry.cpp pins with static_asserts (232 bytes, slot_mapping at 176, tokens at 200, theta at 224)."""
    st = abi.EXTENSION_STRUCTS["RoostQkvQkNormRopeCacheWriteParams"]
    assert C.sizeof(st) == 232
    assert (st.slot_mapping.offset, st.tokens.offset, st.theta.offset) == (176, 200, 224)
    spans = [f[0] for f in st._fields_ if f[1] is abi.DeviceSpan]
    assert spans == ["qkv", "q", "q_weight", "k_weight", "positions", "k_cache", "v_cache", "slot_mapping"]


def declared_symbols():
    syms = set()
    for h in (ROOT / "include").glob("*.h"):
        syms |= set(re.findall(r"ROOST_API\s+[\w\s\*]+?\b(roost_\w+)\s*\(", h.read_text()))
    return syms


def test_library_exports_every_declared_symbol(kernels):
    out = subprocess.run(["nm", "-D", "--defined-only", str(kernels.path)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    declared = declared_symbols()
    assert {"roost_abi_version", "roost_last_error", "roost_register", "roost_context_create",
            "roost_context_destroy", "roost_paged_attention_run", "roost_cache_write_run", "roost_gdn_chunk_run",
            "roost_gdn_recurrent_run", "roost_gated_delta_rule_gates_run", "roost_gated_rms_norm_run",
            "roost_sigmoid_mul_run", "roost_causal_conv1d_run", "roost_recurrent_state_copy_run",
            "roost_recurrent_state_snapshot_run", "roost_qk_norm_run", "roost_rope_run",
            "roost_qkv_qk_norm_rope_cache_write_run"} <= declared
    assert declared <= exported, declared - exported


def test_abi_version_and_table(kernels):
    assert kernels.dll.roost_abi_version() == (1 << 16) | 3
    assert kernels.table.entry_size == 128
    assert kernels.table.library_abi_major == 1 and kernels.table.library_abi_minor == 3
    assert kernels.library_name == "roost-kernels-gfx950"
    ids = {e.variant_id: e for e in kernels.entries}
    # The worker names the recurrent GDN variant by id (reference CudaOps.cs:28).
    assert roost_amd.RECURRENT_VARIANT == "gated-delta-rule-recurrent-aot"
    assert set(ids) == {roost_amd.ATTENTION_VARIANT, roost_amd.CACHE_WRITE_VARIANT, roost_amd.CHUNK_VARIANT,
                        roost_amd.RECURRENT_VARIANT, roost_amd.GATES_VARIANT, roost_amd.GATED_RMS_NORM_VARIANT,
                        roost_amd.SIGMOID_MUL_VARIANT, roost_amd.CAUSAL_CONV1D_VARIANT, roost_amd.STATE_COPY_VARIANT,
                        roost_amd.STATE_SNAPSHOT_VARIANT, roost_amd.QK_NORM_VARIANT, roost_amd.ROPE_VARIANT,
                        roost_amd.QKV_VARIANT}
    # The GDN layer's neighbour ops and the attention input ops: graph capturable, deterministic, batch invariant, no plan, no workspace.
    for vid, op, size in [(roost_amd.GATES_VARIANT, abi.OP_GATED_DELTA_RULE_GATES, 168),
                          (roost_amd.GATED_RMS_NORM_VARIANT, abi.OP_GATED_RMS_NORM, 120),
                          (roost_amd.SIGMOID_MUL_VARIANT, abi.OP_SIGMOID_MUL, 88),
                          (roost_amd.CAUSAL_CONV1D_VARIANT, abi.OP_CAUSAL_CONV1D, 200),
                          (roost_amd.STATE_COPY_VARIANT, abi.OP_RECURRENT_STATE_COPY, 72),
                          (roost_amd.STATE_SNAPSHOT_VARIANT, abi.OP_RECURRENT_STATE_SNAPSHOT, 96),
                          (roost_amd.QK_NORM_VARIANT, abi.OP_QK_NORM, 136), (roost_amd.ROPE_VARIANT, abi.OP_ROPE, 128),
                          (roost_amd.QKV_VARIANT, abi.OP_QKV_QK_NORM_ROPE_CACHE_WRITE, 232)]:
        e = ids[vid]
        assert e.op == op and e.params_struct_size == size and e.plan is None and e.workspace is None
        assert e.flags == abi.FLAG_GRAPH_CAPTURABLE | abi.FLAG_DETERMINISTIC | abi.FLAG_BATCH_INVARIANT
        assert e.constraints.sm_min == 950
    att = ids[roost_amd.ATTENTION_VARIANT]
    assert att.op == abi.OP_PAGED_ATTENTION and att.needs_plan and att.params_struct_size == 296
    assert att.constraints.sm_min == 950 and att.constraints.group_size_mask == (1 << 3) | (1 << 7) | (1 << 15) | (1 << 31)
    assert att.constraints.head_dim_mask & (1 << (256 // 16 - 1))
    cw = ids[roost_amd.CACHE_WRITE_VARIANT]
    assert cw.op == abi.OP_CACHE_WRITE and cw.plan is None and cw.params_struct_size == 160
    rec = ids[roost_amd.RECURRENT_VARIANT]
    assert rec.flags & abi.FLAG_GRAPH_CAPTURABLE and not rec.needs_plan and rec.params_struct_size == 280
    ch = ids[roost_amd.CHUNK_VARIANT]
    assert ch.needs_plan and ch.plan is not None and ch.op == abi.OP_GATED_DELTA_RULE
    for e in kernels.entries:
        assert e.params_abi_minor == 3 and e.flags & ~0x1F == 0


def test_register_rejects_old_or_small_tables(kernels):
    t = abi.OpTable()
    t.struct_size = 16
    t.abi_minor = 3
    assert kernels.dll.roost_register(C.byref(t)) == abi.ABI_MISMATCH
    t = abi.new(abi.OpTable)
    t.abi_minor = 4
    assert kernels.dll.roost_register(C.byref(t)) == abi.ABI_MISMATCH
    assert kernels.dll.roost_register(None) == abi.INVALID_ARGUMENT
    assert kernels.last_error()


def test_context_create_rules(kernels):
    p = abi.new(abi.ContextCreateParams)
    p.reserved0 = 1
    out = C.c_void_p()
    assert kernels.dll.roost_context_create(C.byref(p), C.byref(out)) == abi.INVALID_ARGUMENT
    p = abi.new(abi.ContextCreateParams)
    p.struct_size = 8
    assert kernels.dll.roost_context_create(C.byref(p), C.byref(out)) == abi.ABI_MISMATCH
    ctx = kernels.create_context(0)
    assert ctx.value
    kernels.destroy_context(ctx)


def _fake(n, dtype):
    # Spans whose addresses are never dereferenced: every call below is refused before any launch.
    s = abi.DeviceSpan()
    s.address = 0x10000
    s.length = n
    s.dtype = dtype
    return s


def test_attention_refusals_without_gpu(kernels):
    e = kernels.entry(roost_amd.ATTENTION_VARIANT)
    p = abi.new(abi.PagedAttentionParams)
    p.mode, p.batch, p.tokens, p.q_heads, p.kv_heads, p.head_dim, p.page_size = 0, 2, 2, 8, 2, 256, 16
    p.kv_layout, p.window_left = abi.LAYOUT_PAGED_NHD, -1
    for name in ("q", "output", "k_cache", "v_cache"):
        setattr(p, name, _fake(1 << 20, abi.DTYPE_BF16))
    for name in ("q_indptr", "kv_indptr", "kv_last_page_len", "kv_indices"):
        setattr(p, name, _fake(64, abi.DTYPE_I32))
    ctx = kernels.create_context(0)
    run = lambda q: e.run(ctx, C.addressof(q), None, None)  # noqa: E731
    assert run(p) == abi.NOT_PLANNED  # valid params, no plan record
    for field, value, want in [("head_dim", 96, abi.UNSUPPORTED), ("q_heads", 12, abi.UNSUPPORTED),
                               ("window_left", 0, abi.INVALID_ARGUMENT), ("logits_soft_cap", float("nan"), abi.INVALID_ARGUMENT),
                               ("tokens", 3, abi.INVALID_ARGUMENT), ("mode", 7, abi.INVALID_ARGUMENT),
                               ("kv_layout", 0, abi.INVALID_ARGUMENT), ("batch", 0, abi.INVALID_ARGUMENT),
                               ("struct_size", 64, abi.ABI_MISMATCH), ("abi_minor", 4, abi.ABI_MISMATCH)]:
        q = abi.PagedAttentionParams.from_buffer_copy(p)
        setattr(q, field, value)
        assert run(q) == want, field
        assert kernels.last_error()
    q = abi.PagedAttentionParams.from_buffer_copy(p)
    q.q.dtype = abi.DTYPE_F16
    assert run(q) == abi.INVALID_ARGUMENT
    # Workspace query and plan need the host tables.
    sizes = abi.new(abi.WorkspaceSizes)
    assert e.workspace(ctx, C.addressof(p), C.addressof(sizes)) == abi.INVALID_ARGUMENT
    qi = (C.c_int32 * 3)(0, 1, 2)
    ki = (C.c_int32 * 3)(0, 3, 5)
    last = (C.c_int32 * 2)(16, 0)
    p.q_indptr_host, p.kv_indptr_host, p.kv_last_page_len_host = C.addressof(qi), C.addressof(ki), C.addressof(last)
    assert e.workspace(ctx, C.addressof(p), C.addressof(sizes)) == abi.INVALID_ARGUMENT  # last page length 0
    last[1] = 7
    assert e.workspace(ctx, C.addressof(p), C.addressof(sizes)) == abi.OK
    assert sizes.plan_bytes > 0 and sizes.device_alignment == 256
    kernels.destroy_context(ctx)


def test_gdn_refusals_without_gpu(kernels):
    rec = kernels.entry(roost_amd.RECURRENT_VARIANT)
    p = abi.new(abi.GatedDeltaRuleParams)
    p.batch, p.tokens, p.k_heads, p.v_heads, p.k_dim, p.v_dim, p.l2_norm_qk = 1, 2, 16, 16, 128, 128, 1
    for name in ("q", "k", "v", "output"):
        setattr(p, name, _fake(2 * 2048, abi.DTYPE_BF16))
    p.g = _fake(32, abi.DTYPE_F32)
    p.beta = _fake(32, abi.DTYPE_BF16)
    p.state = _fake(16 * 128 * 128, abi.DTYPE_F32)
    p.state_slots = _fake(1, abi.DTYPE_I32)
    p.cu_seqlens = _fake(2, abi.DTYPE_I32)
    ctx = kernels.create_context(0)
    run = lambda q: rec.run(ctx, C.addressof(q), None, None)  # noqa: E731
    for field, value, want in [("k_heads", 3, abi.UNSUPPORTED), ("k_heads", 1, abi.UNSUPPORTED), ("k_dim", 64, abi.UNSUPPORTED),
                               ("l2_norm_qk", 0, abi.UNSUPPORTED), ("q_stride", 2040, abi.INVALID_ARGUMENT),
                               ("struct_size", 64, abi.ABI_MISMATCH)]:
        q = abi.GatedDeltaRuleParams.from_buffer_copy(p)
        setattr(q, field, value)
        assert run(q) == want, field
    q = abi.GatedDeltaRuleParams.from_buffer_copy(p)
    q.beta.dtype = abi.DTYPE_F32
    assert run(q) == abi.UNSUPPORTED
    q = abi.GatedDeltaRuleParams.from_buffer_copy(p)
    q.state.length += 5
    assert run(q) == abi.INVALID_ARGUMENT
    q = abi.GatedDeltaRuleParams.from_buffer_copy(p)
    q.g.address += 4
    assert run(q) == abi.INVALID_ARGUMENT
    chunk = kernels.entry(roost_amd.CHUNK_VARIANT)
    assert chunk.run(ctx, C.addressof(p), None, None) == abi.WORKSPACE_TOO_SMALL
    # The recurrent variant asks for no workspace while no sequence can reach 16 tokens, and for the chunk tables
    # and records once one can; without them such a call is refused before any launch.
    sizes = abi.new(abi.WorkspaceSizes)
    assert rec.workspace(ctx, C.addressof(p), C.addressof(sizes)) == abi.OK and sizes.device_bytes == 0
    long = abi.GatedDeltaRuleParams.from_buffer_copy(p)
    long.tokens = 40
    for name in ("q", "k", "v", "output"):
        setattr(long, name, _fake(40 * 2048, abi.DTYPE_BF16))
    long.g, long.beta = _fake(40 * 16, abi.DTYPE_F32), _fake(40 * 16, abi.DTYPE_BF16)
    assert rec.workspace(ctx, C.addressof(long), C.addressof(sizes)) == abi.OK
    # 40 tokens in one sequence: at most 40 // 64 + min(1, 40 // 16) = 1 chunk of 16 heads x 20480-byte records.
    assert sizes.device_bytes == 256 + 256 + 16 * 20480 and sizes.pinned_host_bytes == 0 and sizes.plan_bytes == 0
    assert run(long) == abi.WORKSPACE_TOO_SMALL
    kernels.destroy_context(ctx)


def test_product_path_has_no_oracle_or_cpu_fallback():
    """The library and its host package never reach the oracle."""
    for f in list((ROOT / "roost_amd").rglob("*.py")) + list((ROOT / "roost_amd" / "csrc").glob("*")):
        text = f.read_text(errors="ignore")
        assert "import oracle" not in text and "from oracle" not in text and "liboracle" not in text, f
