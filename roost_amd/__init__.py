"""roost_amd -- host side of the MI355X (gfx950) Roost attention + Gated DeltaNet kernel library.

The product is ``libroost_kernels_gfx950.so`` (built from ``roost_amd/csrc`` by ``roost_amd/build.py``), exporting
Roost's C ABI 1.3. This package is the Python mirror of the reference's host interface for that library:

* ``KernelLibrary`` mirrors ``Starlings.Roost.Kernels.KernelLibrary`` (reference src/Starlings.Roost.Kernels/
  KernelLibrary.cs:107-373): load by exports, check the ABI version, read the registration table with its
  ``entry_size`` stride, refuse a NEEDS_PLAN/plan disagreement, create the context;
* ``OpSession`` mirrors ``CudaOpsSession.Launch`` (src/Starlings.Roost.Worker/Eager/CudaOpsSession.cs:184-254): query
  the workspace, (re)allocate it when it does not fit, ``plan()`` when the variant needs one, then ``run()`` on the
  session's stream;
* ``paged_attention``, ``cache_write`` and ``gated_delta_rule`` mirror ``CudaOps.PagedAttention / CacheWrite /
  GatedDeltaRule`` (src/Starlings.Roost.Worker/Eager/CudaOps.cs:106-144, 251-272; CudaOps.Hybrid.cs:9-40): they fill
  the params struct from tensors and pick the variant the worker would pick.

PyTorch is used only for device memory and streams. There is no fallback: if the library is missing or fails to load,
every call raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

from . import abi

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libroost_kernels_gfx950.so"

RECURRENT_VARIANT = "gated-delta-rule-recurrent-aot"
CHUNK_VARIANT = "gated-delta-rule-chunk-gfx950"
ATTENTION_VARIANT = "paged-attention-gfx950"
CACHE_WRITE_VARIANT = "cache-write-gfx950"
GATES_VARIANT = "gated-delta-rule-gates-gfx950"
GATED_RMS_NORM_VARIANT = "gated-rms-norm-gfx950"
SIGMOID_MUL_VARIANT = "sigmoid-mul-gfx950"
CAUSAL_CONV1D_VARIANT = "causal-conv1d-gfx950"
STATE_COPY_VARIANT = "recurrent-state-copy-gfx950"
STATE_SNAPSHOT_VARIANT = "recurrent-state-snapshot-gfx950"
QK_NORM_VARIANT = "qk-norm-gfx950"
ROPE_VARIANT = "rope-gfx950"
QKV_VARIANT = "qkv-qk-norm-rope-cache-write-gfx950"


class KernelError(RuntimeError):
    def __init__(self, op: str, status: int, message: str):
        name = abi.STATUS_NAMES[status] if 0 <= status < len(abi.STATUS_NAMES) else str(status)
        super().__init__(f"{op}: {name} ({status}): {message}")
        self.status = status


@dataclass
class Entry:
    op: int
    flags: int
    variant_id: str
    params_struct_size: int
    params_abi_minor: int
    constraints: abi.Constraints
    run: Optional[abi.RunFn]
    plan: Optional[abi.PlanFn]
    workspace: Optional[abi.WorkspaceFn]

    @property
    def needs_plan(self) -> bool:
        return bool(self.flags & abi.FLAG_NEEDS_PLAN)


class KernelLibrary:
    """The loaded library: exports, registration table and last-error text."""

    EXPORTS = ("roost_abi_version", "roost_last_error", "roost_register", "roost_context_create",
               "roost_context_destroy")

    def __init__(self, path: Path | str = LIB_PATH):
        path = Path(path)
        if not path.exists():
            raise FileNotFoundError(f"{path} is missing: run `python -m roost_amd.build` (or __graft_entry__.build())")
        self.path = path
        # The library must share the process's HIP runtime (streams and device pointers pass between them). In a
        # Python host that runtime is the one PyTorch loads: its libamdhip64 carries the soname libamdhip64.so.7, so
        # loading torch first makes the library's DT_NEEDED entry bind to it instead of a second copy.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        self.dll = C.CDLL(str(path))
        for name in self.EXPORTS:
            if not hasattr(self.dll, name):
                raise RuntimeError(f"{path}: export {name} is missing")
        self.dll.roost_abi_version.restype = C.c_uint32
        self.dll.roost_last_error.restype = C.c_char_p
        self.dll.roost_register.argtypes = [C.POINTER(abi.OpTable)]
        self.dll.roost_register.restype = C.c_int32
        self.dll.roost_context_create.argtypes = [C.POINTER(abi.ContextCreateParams), C.POINTER(C.c_void_p)]
        self.dll.roost_context_create.restype = C.c_int32
        self.dll.roost_context_destroy.argtypes = [C.c_void_p]
        self.dll.roost_context_destroy.restype = C.c_int32
        self.dll.roost_amd_plan_region_fill.argtypes = [C.POINTER(abi.PlanRegion)]
        self.dll.roost_amd_plan_region_fill.restype = C.c_int32
        self.dll.roost_amd_plan_region_run.argtypes = [C.c_void_p, C.POINTER(abi.PlanRegion), C.c_void_p]
        self.dll.roost_amd_plan_region_run.restype = C.c_int32
        self.dll.roost_amd_gdn_recurrent_gated_run.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                               C.c_void_p]
        self.dll.roost_amd_gdn_recurrent_gated_run.restype = C.c_int32
        self.dll.roost_amd_paged_attention_gated_run.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                                 C.c_void_p]
        self.dll.roost_amd_paged_attention_gated_run.restype = C.c_int32
        self.dll.roost_amd_gdn_decode_layer_run.argtypes = [C.c_void_p] * 6
        self.dll.roost_amd_gdn_decode_layer_run.restype = C.c_int32
        self.dll.roost_amd_gdn_chunk_layer_run.argtypes = [C.c_void_p] * 7
        self.dll.roost_amd_gdn_chunk_layer_run.restype = C.c_int32
        self.dll.roost_amd_gdn_chunk_layer_plan.argtypes = [C.c_void_p] * 5
        self.dll.roost_amd_gdn_layer_run.argtypes = [C.c_void_p] * 7
        self.dll.roost_amd_gdn_layer_run.restype = C.c_int32
        self.dll.roost_amd_gdn_chunk_layer_plan.restype = C.c_int32
        self.dll.roost_amd_plan_region_from_step.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(abi.StepTables)]
        self.dll.roost_amd_plan_region_from_step.restype = C.c_int32
        version = self.dll.roost_abi_version()
        if version >> 16 != abi.ABI_MAJOR or (version & 0xFFFF) < abi.ABI_MINOR:
            raise RuntimeError(f"{path}: ABI {version >> 16}.{version & 0xFFFF} is not {abi.ABI_MAJOR}.{abi.ABI_MINOR}")
        self.table = abi.new(abi.OpTable)
        status = self.dll.roost_register(C.byref(self.table))
        if status != abi.OK:
            raise KernelError("roost_register", status, self.last_error())
        self.library_name = self.table.library_name.decode()
        self.entries: list[Entry] = []
        base = self.table.entries
        seen = set()
        for i in range(self.table.entry_count):
            raw = abi.OpEntry.from_address(base + i * self.table.entry_size)
            vid = raw.variant_id.decode()
            if (raw.op, vid) in seen:
                raise RuntimeError(f"duplicate variant {vid}")
            seen.add((raw.op, vid))
            if bool(raw.flags & abi.FLAG_NEEDS_PLAN) != bool(raw.plan):
                raise RuntimeError(f"variant {vid}: NEEDS_PLAN and the plan entry point disagree")
            self.entries.append(Entry(
                raw.op, raw.flags, vid, raw.params_struct_size, raw.params_abi_minor, raw.constraints,
                abi.RunFn(raw.run) if raw.run else None, abi.PlanFn(raw.plan) if raw.plan else None,
                abi.WorkspaceFn(raw.workspace) if raw.workspace else None))

    def last_error(self) -> str:
        return self.dll.roost_last_error().decode(errors="replace")

    def entry(self, variant_id: str) -> Entry:
        for e in self.entries:
            if e.variant_id == variant_id:
                return e
        raise KeyError(f"variant {variant_id} is not registered by {self.library_name}")

    def create_context(self, device: int = 0, flags: int = 0) -> C.c_void_p:
        p = abi.new(abi.ContextCreateParams)
        p.device = device
        p.flags = flags
        ctx = C.c_void_p()
        status = self.dll.roost_context_create(C.byref(p), C.byref(ctx))
        if status != abi.OK:
            raise KernelError("roost_context_create", status, self.last_error())
        return ctx

    def destroy_context(self, ctx: C.c_void_p) -> None:
        self.dll.roost_context_destroy(ctx)


_LIBRARY: Optional[KernelLibrary] = None


def library() -> KernelLibrary:
    """The process-wide library (loaded on first use; raises if it is not built)."""
    global _LIBRARY
    if _LIBRARY is None:
        _LIBRARY = KernelLibrary()
    return _LIBRARY


# ---- tensors -> spans -------------------------------------------------------------------------------------------------

def _torch():
    import torch  # noqa: WPS433 -- torch is plumbing for device memory and streams
    return torch


def dtype_of(t) -> int:
    torch = _torch()
    return {torch.float32: abi.DTYPE_F32, torch.float16: abi.DTYPE_F16, torch.bfloat16: abi.DTYPE_BF16,
            torch.float64: abi.DTYPE_F64, torch.int32: abi.DTYPE_I32, torch.int64: abi.DTYPE_I64,
            torch.uint8: abi.DTYPE_U8}[t.dtype]


def span(t, *, length: Optional[int] = None, dtype: Optional[int] = None, offset_elems: int = 0) -> abi.DeviceSpan:
    """A RoostDeviceSpan over tensor t (optionally a sub-range starting offset_elems in)."""
    s = abi.DeviceSpan()
    if t is None:
        return s
    s.address = t.data_ptr() + offset_elems * t.element_size()
    s.length = t.numel() - offset_elems if length is None else length
    s.dtype = dtype_of(t) if dtype is None else dtype
    return s


def host_ptr(a) -> Optional[int]:
    """Address of a host (numpy or CPU tensor) int32 table, or None."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        assert not a.is_cuda
        return a.data_ptr()
    return a.ctypes.data


class OpSession:
    """One context + stream: workspace query, allocation, plan and run, as the worker's CudaOpsSession does."""

    def __init__(self, lib: Optional[KernelLibrary] = None, device: int = 0, stream=None):
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError("OpSession needs a GPU (the gfx950 library has no CPU path)")
        self.lib = lib or library()
        self.device = torch.device("cuda", device)
        self.stream = stream or torch.cuda.current_stream(self.device)
        self.ctx = self.lib.create_context(device)
        self._ws = {}  # (variant, key) -> [device tensor, pinned tensor, plan buffer, Workspace, event]

    @property
    def stream_handle(self) -> int:
        return self.stream.cuda_stream

    def workspace_sizes(self, entry: Entry, params) -> abi.WorkspaceSizes:
        sizes = abi.new(abi.WorkspaceSizes)
        if entry.workspace is not None:
            status = entry.workspace(self.ctx, C.addressof(params), C.addressof(sizes))
            if status != abi.OK:
                raise KernelError(f"{entry.variant_id} workspace", status, self.lib.last_error())
        return sizes

    def _workspace(self, entry: Entry, params, key) -> abi.Workspace:
        torch = _torch()
        sizes = self.workspace_sizes(entry, params)
        slot = self._ws.get((entry.variant_id, key))
        fits = slot is not None and slot[3].device_bytes >= sizes.device_bytes and \
            slot[3].pinned_host_bytes >= sizes.pinned_host_bytes and slot[3].plan_bytes >= sizes.plan_bytes
        if not fits:
            self.stream.synchronize()  # in-flight kernels may still read the old buffers
            dev = torch.empty(max(int(sizes.device_bytes), 1) + 256, dtype=torch.uint8, device=self.device)
            pinned = torch.empty(max(int(sizes.pinned_host_bytes), 1), dtype=torch.uint8, pin_memory=True)
            plan = C.create_string_buffer(max(int(sizes.plan_bytes), 1))
            ws = abi.new(abi.Workspace)
            base = dev.data_ptr()
            ws.device = (base + 255) // 256 * 256
            ws.device_bytes = sizes.device_bytes
            ws.pinned_host = pinned.data_ptr()
            ws.pinned_host_bytes = sizes.pinned_host_bytes
            ws.plan = C.addressof(plan)
            ws.plan_bytes = sizes.plan_bytes
            slot = [dev, pinned, plan, ws, None]
            self._ws[(entry.variant_id, key)] = slot
        return slot

    def prepare(self, entry: Entry, params, key=0, plan: bool = True) -> Optional[abi.Workspace]:
        """Workspace -> (plan) on the session stream; the workspace a run() of these params takes (None: none)."""
        if entry.workspace is None:
            return None
        slot = self._workspace(entry, params, key)
        ws = slot[3]
        if entry.needs_plan and plan:
            if slot[4] is not None:
                slot[4].synchronize()  # the previous plan's host->device copy has left the pinned buffer
            status = entry.plan(self.ctx, C.addressof(params), C.addressof(ws), C.c_void_p(self.stream_handle))
            if status != abi.OK:
                raise KernelError(f"{entry.variant_id} plan", status, self.lib.last_error())
            ev = _torch().cuda.Event()
            ev.record(self.stream)
            slot[4] = ev
        return ws

    def launch(self, entry: Entry, params, key=0, plan: bool = True) -> None:
        """Workspace -> (plan) -> run on the session stream."""
        self.run(entry, params, self.prepare(entry, params, key, plan))

    def run(self, entry: Entry, params, ws: Optional[abi.Workspace]) -> None:
        status = self.run_raw(entry, params, ws)
        if status != abi.OK:
            raise KernelError(f"{entry.variant_id} run", status, self.lib.last_error())

    def run_raw(self, entry: Entry, params, ws: Optional[abi.Workspace]) -> int:
        return entry.run(self.ctx, C.addressof(params), C.addressof(ws) if ws is not None else None,
                         C.c_void_p(self.stream_handle))

    def close(self) -> None:
        if self.ctx:
            self.stream.synchronize()
            self.lib.destroy_context(self.ctx)
            self.ctx = None
            self._ws.clear()


# ---- op mirrors (CudaOps) ---------------------------------------------------------------------------------------------

def paged_attention_params(q, output, k_cache, v_cache, q_indptr, kv_indptr, kv_indices, kv_last_page_len, *,
                           q_indptr_host, kv_indptr_host, kv_last_page_len_host, batch, q_heads, kv_heads, head_dim,
                           page_size, kv_layout=abi.LAYOUT_PAGED_NHD, sm_scale=0.0, causal=True, lse=None,
                           mode=None, window_left=-1, soft_cap=0.0):
    """Fills RoostPagedAttentionParams as CudaOps.PagedAttention does: prefill whenever tokens > batch."""
    tokens = q.shape[0]
    p = abi.new(abi.PagedAttentionParams)
    p.q, p.output, p.lse = span(q), span(output), span(lse)
    p.k_cache, p.v_cache = span(k_cache), span(v_cache)
    p.q_indptr, p.kv_indptr, p.kv_indices = span(q_indptr), span(kv_indptr), span(kv_indices)
    p.kv_last_page_len = span(kv_last_page_len)
    p.q_indptr_host = host_ptr(q_indptr_host)
    p.kv_indptr_host = host_ptr(kv_indptr_host)
    p.kv_last_page_len_host = host_ptr(kv_last_page_len_host)
    p.mode = (abi.ATTENTION_PREFILL if tokens > batch else abi.ATTENTION_DECODE) if mode is None else mode
    p.batch, p.tokens = batch, tokens
    p.q_heads, p.kv_heads, p.head_dim = q_heads, kv_heads, head_dim
    p.page_size, p.kv_layout = page_size, kv_layout
    p.sm_scale, p.logits_soft_cap, p.window_left, p.causal = sm_scale, soft_cap, window_left, int(causal)
    # The struct holds raw addresses: keep every buffer it points at alive for as long as the struct is.
    p._keep = (q, output, lse, k_cache, v_cache, q_indptr, kv_indptr, kv_indices, kv_last_page_len, q_indptr_host,
               kv_indptr_host, kv_last_page_len_host)
    return p


def paged_attention(session: OpSession, *args, **kwargs) -> None:
    p = paged_attention_params(*args, **kwargs)
    session.launch(session.lib.entry(ATTENTION_VARIANT), p, key=(p.mode, p.batch, p.tokens))


def cache_write_params(k, v, k_cache, v_cache, slot_mapping, *, kv_heads, head_dim, page_size,
                       kv_layout=abi.LAYOUT_PAGED_NHD):
    p = abi.new(abi.CacheWriteParams)
    p.k, p.v, p.k_cache, p.v_cache, p.slot_mapping = span(k), span(v), span(k_cache), span(v_cache), span(slot_mapping)
    p.tokens = k.shape[0]
    p.kv_heads, p.head_dim, p.page_size, p.kv_layout = kv_heads, head_dim, page_size, kv_layout
    p.k_scale = p.v_scale = 1.0
    p._keep = (k, v, k_cache, v_cache, slot_mapping)
    return p


def cache_write(session: OpSession, *args, **kwargs) -> None:
    p = cache_write_params(*args, **kwargs)
    session.launch(session.lib.entry(CACHE_WRITE_VARIANT), p)


def gated_delta_rule_params(q, k, v, g, beta, output, state, state_slots, cu_seqlens, *, batch, tokens, k_heads=16,
                            v_heads=16, k_dim=128, v_dim=128, q_stride=0, k_stride=0, v_stride=0,
                            use_initial_state=True, l2_norm_qk=True, scale=0.0, cu_seqlens_host=None,
                            q_len=None, k_len=None, v_len=None, q_offset=0, k_offset=0, v_offset=0):
    """Fills RoostGatedDeltaRuleParams. q/k/v may be column views of one fused tensor (offset + stride)."""
    p = abi.new(abi.GatedDeltaRuleParams)
    p.q = span(q, length=q_len, offset_elems=q_offset)
    p.k = span(k, length=k_len, offset_elems=k_offset)
    p.v = span(v, length=v_len, offset_elems=v_offset)
    p.g, p.beta, p.output = span(g), span(beta), span(output)
    p.state, p.state_slots, p.cu_seqlens = span(state), span(state_slots), span(cu_seqlens)
    p.cu_seqlens_host = host_ptr(cu_seqlens_host)
    p.batch, p.tokens = batch, tokens
    p.k_heads, p.v_heads, p.k_dim, p.v_dim = k_heads, v_heads, k_dim, v_dim
    p.q_stride, p.k_stride, p.v_stride = q_stride, k_stride, v_stride
    p.use_initial_state, p.l2_norm_qk, p.scale = int(use_initial_state), int(l2_norm_qk), scale
    p._keep = (q, k, v, g, beta, output, state, state_slots, cu_seqlens, cu_seqlens_host)
    return p


def gated_delta_rule(session: OpSession, *args, variant: str = RECURRENT_VARIANT, **kwargs) -> None:
    """CudaOps.GatedDeltaRule runs the recurrent variant for every length; the chunk variant is selectable."""
    p = gated_delta_rule_params(*args, **kwargs)
    session.launch(session.lib.entry(variant), p, key=(p.batch, p.tokens))


# ---- the GDN layer's neighbour ops (CudaOps.GatedDeltaRuleGates / GatedRmsNorm / SigmoidMul / CausalConv1d and the
# recurrent-state copies) ----------------------------------------------------------------------------------------------

def gated_delta_rule_gates_params(a, b, a_log, dt_bias, g, beta, *, tokens, v_heads, a_stride=0, b_stride=0,
                                  a_len=None, b_len=None, a_offset=0, b_offset=0):
    """Fills RoostGatedDeltaRuleGatesParams; a and b may be column views of one projection (offset + stride)."""
    p = abi.new(abi.GatedDeltaRuleGatesParams)
    p.a = span(a, length=a_len, offset_elems=a_offset)
    p.b = span(b, length=b_len, offset_elems=b_offset)
    p.a_log, p.dt_bias, p.g, p.beta = span(a_log), span(dt_bias), span(g), span(beta)
    p.tokens, p.v_heads, p.a_stride, p.b_stride = tokens, v_heads, a_stride, b_stride
    p._keep = (a, b, a_log, dt_bias, g, beta)
    return p


def gated_rms_norm_params(x, gate, weight, out, *, rows, dim, eps):
    p = abi.new(abi.GatedRmsNormParams)
    p.input, p.gate, p.weight, p.output = span(x), span(gate), span(weight), span(out)
    p.rows, p.dim, p.eps = rows, dim, eps
    p._keep = (x, gate, weight, out)
    return p


def qk_norm_params(q, k, q_weight, k_weight, *, tokens, q_heads, kv_heads, head_dim, eps, q_stride=0, k_stride=0):
    """RoostQkNormParams: per-head RmsNorm of q and k in place (q_stride / k_stride: elements between tokens)."""
    p = abi.new(abi.QkNormParams)
    p.q, p.k, p.q_weight, p.k_weight = span(q), span(k), span(q_weight), span(k_weight)
    p.tokens, p.q_heads, p.kv_heads, p.head_dim = tokens, q_heads, kv_heads, head_dim
    p.q_stride, p.k_stride, p.eps = q_stride, k_stride, eps
    p._keep = (q, k, q_weight, k_weight)
    return p


def rope_params(q, k, positions, *, tokens, q_heads, kv_heads, head_dim, theta, rotary_dim=0, interleaved=False,
                llama3=None):
    """RoostRopeParams; llama3 = (factor, low_freq_factor, high_freq_factor, original_max_position) selects Llama 3."""
    p = abi.new(abi.RopeParams)
    p.q, p.k, p.positions = span(q), span(k), span(positions)
    p.tokens, p.q_heads, p.kv_heads, p.head_dim = tokens, q_heads, kv_heads, head_dim
    p.rotary_dim, p.interleaved, p.theta = rotary_dim, int(interleaved), theta
    if llama3 is not None:
        p.kind = abi.ROPE_LLAMA3
        (p.llama3_factor, p.llama3_low_freq_factor, p.llama3_high_freq_factor,
         p.llama3_original_max_position) = llama3
    p._keep = (q, k, positions)
    return p


def qkv_qk_norm_rope_cache_write_params(qkv, q, q_weight, k_weight, positions, k_cache, v_cache, slot_mapping, *,
                                        tokens, q_heads, kv_heads, head_dim, page_size, eps, theta):
    """RoostQkvQkNormRopeCacheWriteParams (QkvQkNormRopeCacheWriteArgs of the reference's C# ops)."""
    p = abi.new(abi.QkvQkNormRopeCacheWriteParams)
    p.qkv, p.q, p.q_weight, p.k_weight, p.positions = span(qkv), span(q), span(q_weight), span(k_weight), span(positions)
    p.k_cache, p.v_cache, p.slot_mapping = span(k_cache), span(v_cache), span(slot_mapping)
    p.tokens, p.q_heads, p.kv_heads, p.head_dim, p.page_size = tokens, q_heads, kv_heads, head_dim, page_size
    p.eps, p.theta = eps, theta
    p._keep = (qkv, q, q_weight, k_weight, positions, k_cache, v_cache, slot_mapping)
    return p


def sigmoid_mul_params(x, gate, out, *, rows, dim):
    p = abi.new(abi.SigmoidMulParams)
    p.input, p.gate, p.output = span(x), span(gate), span(out)
    p.rows, p.dim = rows, dim
    p._keep = (x, gate, out)
    return p


def causal_conv1d_params(x, weight, bias, out, conv_state, state_slots, cu_seqlens, *, batch, tokens, channels, width,
                         silu=True):
    p = abi.new(abi.CausalConv1dParams)
    p.input, p.weight, p.bias, p.output = span(x), span(weight), span(bias), span(out)
    p.conv_state, p.state_slots, p.cu_seqlens = span(conv_state), span(state_slots), span(cu_seqlens)
    p.batch, p.tokens, p.channels, p.width, p.silu = batch, tokens, channels, width, int(silu)
    p._keep = (x, weight, bias, out, conv_state, state_slots, cu_seqlens)
    return p


def recurrent_state_copy_params(pool, pairs, *, slot_bytes, count):
    p = abi.new(abi.RecurrentStateCopyParams)
    p.pool, p.pairs, p.slot_bytes, p.count = span(pool), span(pairs), slot_bytes, count
    p._keep = (pool, pairs)
    return p


def recurrent_state_snapshot_params(pool, snapshots, pairs, *, slot_bytes, count, restore):
    p = abi.new(abi.RecurrentStateSnapshotParams)
    p.pool, p.snapshots, p.pairs = span(pool), span(snapshots), span(pairs)
    p.slot_bytes, p.count, p.restore = slot_bytes, count, int(restore)
    p._keep = (pool, snapshots, pairs)
    return p


def gated_delta_rule_gates(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(GATES_VARIANT), gated_delta_rule_gates_params(*args, **kwargs))


def gdn_recurrent_gated(session: OpSession, gdn_params, gates_params, key="gated") -> None:
    """roost_amd_gdn_recurrent_gated_run: the recurrent GatedDeltaRule with the gates computed in its kernels, in the
    recurrent variant's workspace (sized and kept by the session under `key`)."""
    entry = session.lib.entry(RECURRENT_VARIANT)
    ws = session._workspace(entry, gdn_params, key)[3]
    status = session.lib.dll.roost_amd_gdn_recurrent_gated_run(session.ctx, C.addressof(gdn_params),
                                                               C.addressof(gates_params), C.addressof(ws),
                                                               C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("gdn_recurrent_gated", status, session.lib.last_error())


def paged_attention_gated(session: OpSession, attn_params, gate_params, key="gated", plan: bool = True) -> None:
    """roost_amd_paged_attention_gated_run: PagedAttention with the SigmoidMul output gate folded into its kernels, in
    the attention variant's workspace (planned here unless plan is False; sized and kept by the session under key)."""
    entry = session.lib.entry(ATTENTION_VARIANT)
    slot = session._workspace(entry, attn_params, key)
    ws = slot[3]
    if plan:
        if slot[4] is not None:
            slot[4].synchronize()
        status = entry.plan(session.ctx, C.addressof(attn_params), C.addressof(ws), C.c_void_p(session.stream_handle))
        if status != abi.OK:
            raise KernelError(f"{entry.variant_id} plan", status, session.lib.last_error())
        ev = _torch().cuda.Event()
        ev.record(session.stream)
        slot[4] = ev
    status = session.lib.dll.roost_amd_paged_attention_gated_run(session.ctx, C.addressof(attn_params),
                                                                 C.addressof(gate_params), C.addressof(ws),
                                                                 C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("paged_attention_gated", status, session.lib.last_error())


def gdn_decode_layer(session: OpSession, conv_params, gates_params, gdn_params, norm_params) -> None:
    """roost_amd_gdn_decode_layer_run: CausalConv1d, GatedDeltaRuleGates (gates_params may be None: g and beta are then
    read from gdn_params), the recurrent GatedDeltaRule and GatedRmsNorm of one decode step in one call."""
    status = session.lib.dll.roost_amd_gdn_decode_layer_run(
        session.ctx, C.addressof(conv_params), C.addressof(gates_params) if gates_params is not None else None,
        C.addressof(gdn_params), C.addressof(norm_params), C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("gdn_decode_layer", status, session.lib.last_error())


def gdn_layer(session: OpSession, conv_params, gates_params, gdn_params, norm_params, key=0) -> None:
    """roost_amd_gdn_layer_run: CausalConv1d, GatedDeltaRuleGates (gates_params may be None), the recurrent
    GatedDeltaRule and GatedRmsNorm of any step in one call, in the recurrent variant's workspace."""
    ws = session.prepare(session.lib.entry(RECURRENT_VARIANT), gdn_params, ("layer", key), plan=False)
    status = session.lib.dll.roost_amd_gdn_layer_run(
        session.ctx, C.addressof(conv_params), C.addressof(gates_params) if gates_params is not None else None,
        C.addressof(gdn_params), C.addressof(norm_params), C.addressof(ws) if ws is not None else None,
        C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("gdn_layer", status, session.lib.last_error())


def gdn_chunk_layer(session: OpSession, conv_params, gates_params, gdn_params, norm_params, key=0,
                    plan: bool = True) -> None:
    """roost_amd_gdn_chunk_layer_run: CausalConv1d (folded into the chunk prep), GatedDeltaRuleGates (gates_params may
    be None), the chunked GatedDeltaRule and GatedRmsNorm of one prefill pass, in the chunk variant's workspace
    (planned here by roost_amd_gdn_chunk_layer_plan unless plan is False)."""
    chunk = session.lib.entry(CHUNK_VARIANT)
    ws = session.prepare(chunk, gdn_params, ("chunk-layer", key), plan=False)  # the workspace: the chunk variant's
    if plan:
        status = session.lib.dll.roost_amd_gdn_chunk_layer_plan(
            session.ctx, C.addressof(gates_params) if gates_params is not None else None, C.addressof(gdn_params),
            C.addressof(ws), C.c_void_p(session.stream_handle))
        if status != abi.OK:
            raise KernelError("gdn_chunk_layer plan", status, session.lib.last_error())
        session.stream.synchronize()  # the pinned tables are reused by the next plan
    status = session.lib.dll.roost_amd_gdn_chunk_layer_run(
        session.ctx, C.addressof(conv_params), C.addressof(gates_params) if gates_params is not None else None,
        C.addressof(gdn_params), C.addressof(norm_params), C.addressof(ws), C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("gdn_chunk_layer", status, session.lib.last_error())


def gated_rms_norm(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(GATED_RMS_NORM_VARIANT), gated_rms_norm_params(*args, **kwargs))


def sigmoid_mul(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(SIGMOID_MUL_VARIANT), sigmoid_mul_params(*args, **kwargs))


def causal_conv1d(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(CAUSAL_CONV1D_VARIANT), causal_conv1d_params(*args, **kwargs))


def qk_norm(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(QK_NORM_VARIANT), qk_norm_params(*args, **kwargs))


def rope(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(ROPE_VARIANT), rope_params(*args, **kwargs))


def qkv_qk_norm_rope_cache_write(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(QKV_VARIANT), qkv_qk_norm_rope_cache_write_params(*args, **kwargs))


def recurrent_state_copy(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(STATE_COPY_VARIANT), recurrent_state_copy_params(*args, **kwargs))


def recurrent_state_snapshot(session: OpSession, *args, **kwargs) -> None:
    session.launch(session.lib.entry(STATE_SNAPSHOT_VARIANT), recurrent_state_snapshot_params(*args, **kwargs))


# ---- plan region (PlanRegionWriter.Fill) ------------------------------------------------------------------------------

PLAN_REGION_INPUTS = ("token_start", "token_count", "position_offset", "kv_length", "block_indptr", "blocks",
                      "recurrent_slot")
PLAN_REGION_OUTPUTS = ("q_indptr", "cu_seqlens", "kv_indptr", "kv_indices", "kv_last_page_len", "state_slots",
                       "positions", "slot_mapping")


def _address(a) -> Optional[int]:
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data


def plan_region_struct(*, batch: int, tokens: int, block_size: int, **arrays) -> abi.PlanRegion:
    """RoostAmdPlanRegion over numpy arrays (host) or torch tensors (device); absent names are NULL."""
    r = abi.PlanRegion()
    r.batch, r.tokens, r.block_size = batch, tokens, block_size
    for name, a in arrays.items():
        if name not in PLAN_REGION_INPUTS + PLAN_REGION_OUTPUTS:
            raise TypeError(f"unknown plan region array {name}")
        setattr(r, name, _address(a))
    return r


def plan_region_fill(lib: KernelLibrary, **kwargs) -> None:
    """roost_amd_plan_region_fill on host arrays; raises KernelError on a refused plan."""
    r = plan_region_struct(**kwargs)
    status = lib.dll.roost_amd_plan_region_fill(C.byref(r))
    if status != abi.OK:
        raise KernelError("plan_region_fill", status, lib.last_error())


def plan_region_run(session: OpSession, **kwargs) -> None:
    """roost_amd_plan_region_run on device tensors, on the session's stream."""
    r = plan_region_struct(**kwargs)
    status = session.lib.dll.roost_amd_plan_region_run(session.ctx, C.byref(r), C.c_void_p(session.stream_handle))
    if status != abi.OK:
        raise KernelError("plan_region_run", status, session.lib.last_error())


def plan_region_from_step(lib: KernelLibrary, plan, *, attention_group: int, block_size: int, attention_blocks: int,
                          max_batch: int, max_tokens: int, max_blocks: int) -> dict:
    """roost_amd_plan_region_from_step over a C2 step-plan buffer (bytes or a uint8 numpy array). Returns the tables as
    numpy arrays cut to what was written; raises KernelError on a refused plan."""
    import numpy as np

    buf = np.frombuffer(bytes(plan), dtype=np.uint8).copy() if not isinstance(plan, np.ndarray) else plan
    out = {
        "q_indptr": np.full(max_batch + 1, -7, np.int32), "cu_seqlens": np.full(max_batch + 1, -7, np.int32),
        "kv_indptr": np.full(max_batch + 1, -7, np.int32), "kv_indices": np.full(max(max_blocks, 1), -7, np.int32),
        "kv_last_page_len": np.full(max(max_batch, 1), -7, np.int32), "state_slots": np.full(max(max_batch, 1), -7, np.int32),
        "ids": np.full(max(max_tokens, 1), -7, np.int32), "positions": np.full(max(max_tokens, 1), -7, np.int32),
        "slot_mapping": np.full(max(max_tokens, 1), -7, np.int64), "rows": np.full(max(max_batch, 1), -7, np.int32),
    }
    t = abi.StepTables()
    t.attention_group, t.block_size, t.attention_blocks = attention_group, block_size, attention_blocks
    t.max_batch, t.max_tokens, t.max_blocks = max_batch, max_tokens, max_blocks
    for name, a in out.items():
        setattr(t, name, a.ctypes.data)
    status = lib.dll.roost_amd_plan_region_from_step(C.c_void_p(buf.ctypes.data), buf.size, C.byref(t))
    if status != abi.OK:
        raise KernelError("plan_region_from_step", status, lib.last_error())
    n, m, k, r = t.batch, t.tokens, t.blocks, t.rows_written
    return {"q_indptr": out["q_indptr"][:n + 1], "cu_seqlens": out["cu_seqlens"][:n + 1],
            "kv_indptr": out["kv_indptr"][:n + 1], "kv_indices": out["kv_indices"][:k],
            "kv_last_page_len": out["kv_last_page_len"][:n], "state_slots": out["state_slots"][:n],
            "ids": out["ids"][:m], "positions": out["positions"][:m], "slot_mapping": out["slot_mapping"][:m],
            "rows": out["rows"][:r]}
