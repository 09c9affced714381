"""TEST INFRASTRUCTURE ONLY: the parity oracle for the attention + Gated DeltaNet path.

A ctypes binding of ``cpuops.c``, the plain-C restatement of Roost's CpuOps reference (double precision, one rounding
per output element). Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the reported CPU baseline -- never as the thing measured or shipped.

Functions and the reference code they restate:
  paged_attention  -- src/Starlings.Roost.Ops/CpuOps.cs:198-351
  cache_write      -- src/Starlings.Roost.Ops/CpuOps.cs:515-569
  gated_delta_rule -- src/Starlings.Roost.Ops/CpuOps.Hybrid.cs:30-157
  plan_region      -- src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64
  to_bf16          -- src/Starlings.Roost.Ops/CpuElements.cs:128-160
  gdn_gates        -- src/Starlings.Roost.Ops/CpuOps.Gating.cs:21-47
  gated_rms_norm   -- src/Starlings.Roost.Ops/CpuOps.Gating.cs:57-86
  sigmoid_mul      -- src/Starlings.Roost.Ops/CpuOps.Gating.cs:91-101
  causal_conv1d    -- src/Starlings.Roost.Ops/CpuOps.Hybrid.cs:167-243
  state_copy / state_snapshot -- src/Starlings.Roost.Ops/CpuOps.Hybrid.cs:251-263
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_cpuops.so"

DT_F32, DT_BF16, DT_F64, DT_I32, DT_I64 = 1, 3, 4, 10, 12


class OracleError(ValueError):
    """CpuOps would have thrown an ArgumentException for these arguments."""


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_last_error.restype = ctypes.c_char_p
        _lib.oracle_to_bf16.restype = ctypes.c_uint16
        _lib.oracle_to_bf16.argtypes = [ctypes.c_double]
        _lib.oracle_from_bf16.restype = ctypes.c_double
        _lib.oracle_from_bf16.argtypes = [ctypes.c_uint16]
    return _lib


def _ptr(a: np.ndarray | None) -> ctypes.c_void_p:
    if a is None:
        return ctypes.c_void_p(0)
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(lib().oracle_last_error().decode())


def dtype_code(a: np.ndarray, bf16: bool = False) -> int:
    if bf16:
        assert a.dtype == np.uint16
        return DT_BF16
    return {np.dtype(np.float32): DT_F32, np.dtype(np.float64): DT_F64}[a.dtype]


def to_bf16(x) -> np.ndarray:
    """double -> bf16 bits, CpuElements.ToBFloat16 (round-to-odd to float, then nearest even)."""
    f = lib().oracle_to_bf16
    arr = np.asarray(x, dtype=np.float64)
    return np.array([f(float(v)) for v in arr.ravel()], dtype=np.uint16).reshape(arr.shape)


def bf16_to_f64(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits with round-to-nearest-even (vectorised; exact for float32 inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def paged_attention(q, out, k_cache, v_cache, q_indptr, kv_indptr, kv_indices, kv_last_page_len, *, batch, tokens,
                    q_heads, kv_heads, head_dim, page_size, hnd=False, scale=0.0, soft_cap=0.0, window_left=-1,
                    causal=True, bf16=False, threads=1) -> None:
    """CpuOps.PagedAttention. q/out/k_cache/v_cache: float32, float64 or (bf16=True) uint16 bit arrays."""
    dt = dtype_code(q, bf16)
    rc = lib().oracle_paged_attention(
        _ptr(q), _ptr(out), _ptr(k_cache), _ptr(v_cache), dt, dt,
        _ptr(q_indptr), _ptr(kv_indptr), _ptr(kv_indices), _ptr(kv_last_page_len),
        ctypes.c_int64(kv_indices.size), ctypes.c_int64(k_cache.size),
        batch, tokens, q_heads, kv_heads, head_dim, page_size, int(hnd), ctypes.c_float(scale),
        ctypes.c_float(soft_cap), window_left, int(causal), threads)
    _check(rc)


def cache_write(k, v, k_cache, v_cache, slot_mapping, *, tokens, kv_heads, head_dim, page_size, hnd=False,
                bf16=False) -> None:
    """CpuOps.CacheWrite for equal activation and cache types (a byte copy)."""
    dt = dtype_code(k, bf16)
    rc = lib().oracle_cache_write(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), dt, _ptr(slot_mapping),
                                  ctypes.c_int64(k_cache.size), tokens, kv_heads, head_dim, page_size, int(hnd))
    _check(rc)


def gated_delta_rule(q, k, v, g, beta, out, state, state_slots, cu_seqlens, *, batch, tokens, k_heads, v_heads,
                     k_dim, v_dim, q_stride=0, k_stride=0, v_stride=0, use_initial_state=True, l2_norm_qk=True,
                     scale=0.0, bf16=False, g_bf16=False, beta_bf16=False, threads=1) -> None:
    """CpuOps.GatedDeltaRule. state: float32 pool, updated in place."""
    dt = dtype_code(q, bf16)
    rc = lib().oracle_gated_delta_rule(
        _ptr(q), _ptr(k), _ptr(v), _ptr(g), dtype_code(g, g_bf16), _ptr(beta), dtype_code(beta, beta_bf16),
        _ptr(out), _ptr(state), ctypes.c_int64(state.size), _ptr(state_slots), _ptr(cu_seqlens), dt,
        batch, tokens, k_heads, v_heads, k_dim, v_dim, ctypes.c_int64(q_stride), ctypes.c_int64(k_stride),
        ctypes.c_int64(v_stride), int(use_initial_state), int(l2_norm_qk), ctypes.c_float(scale), threads)
    _check(rc)


def _dt(a: np.ndarray) -> int:
    """Element type of an oracle array: uint16 bit arrays are bf16."""
    return {np.dtype(np.float32): DT_F32, np.dtype(np.float64): DT_F64, np.dtype(np.uint16): DT_BF16}[a.dtype]


def gdn_gates(a, b, a_log, dt_bias, g, beta, *, tokens, v_heads, a_stride=0, b_stride=0) -> None:
    """CpuOps.GatedDeltaRuleGates. a and b share one element type; every other array is read or written in its own."""
    assert a.dtype == b.dtype
    _check(lib().oracle_gdn_gates(_ptr(a), _ptr(b), _dt(a), _ptr(a_log), _dt(a_log), _ptr(dt_bias), _dt(dt_bias),
                                  _ptr(g), _dt(g), _ptr(beta), _dt(beta), tokens, v_heads, ctypes.c_int64(a_stride),
                                  ctypes.c_int64(b_stride)))


def gated_rms_norm(x, gate, weight, out, *, rows, dim, eps) -> None:
    """CpuOps.GatedRmsNorm (norm before gate; the weight multiplies as stored)."""
    _check(lib().oracle_gated_rms_norm(_ptr(x), _ptr(gate), _ptr(weight), _dt(weight), _ptr(out), _dt(x),
                                       ctypes.c_int64(rows), dim, ctypes.c_float(eps)))


def sigmoid_mul(x, gate, out) -> None:
    """CpuOps.SigmoidMul over x.size elements."""
    _check(lib().oracle_sigmoid_mul(_ptr(x), _ptr(gate), _ptr(out), _dt(x), ctypes.c_int64(x.size)))


def causal_conv1d(x, weight, bias, out, state, state_slots, cu_seqlens, *, batch, tokens, channels, width,
                  silu) -> None:
    """CpuOps.CausalConv1d; state: the conv-state pool [slots, channels, width - 1], updated in place."""
    _check(lib().oracle_causal_conv1d(_ptr(x), _ptr(weight), _ptr(bias), _ptr(out), _dt(x), _ptr(state), _dt(state),
                                      ctypes.c_int64(state.size), _ptr(state_slots), _ptr(cu_seqlens), batch, tokens,
                                      channels, width, int(silu)))


def qk_norm(q, k, q_weight, k_weight, *, tokens, q_heads, kv_heads, head_dim, eps, q_stride=0, k_stride=0) -> None:
    """CpuOps.QkNorm, in place (q_stride / k_stride: elements between tokens, 0 = contiguous)."""
    assert q.dtype == k.dtype == q_weight.dtype == k_weight.dtype
    qs, ks = q_stride or q_heads * head_dim, k_stride or kv_heads * head_dim
    assert q.size >= (tokens - 1) * qs + q_heads * head_dim and k.size >= (tokens - 1) * ks + kv_heads * head_dim
    assert q_weight.size >= head_dim and k_weight.size >= head_dim
    _check(lib().oracle_qk_norm(_ptr(q), _ptr(k), _ptr(q_weight), _ptr(k_weight), _dt(q), tokens, q_heads, kv_heads,
                                head_dim, q_stride, k_stride, ctypes.c_float(eps)))


def rope(q, k, positions, *, tokens, q_heads, kv_heads, head_dim, theta, rotary_dim=0, interleaved=False,
         llama3=None) -> None:
    """CpuOps.Rope, in place. llama3: (factor, low_freq_factor, high_freq_factor, original_max_position) or None."""
    assert q.dtype == k.dtype and positions.dtype == np.int32
    assert q.size >= tokens * q_heads * head_dim and k.size >= tokens * kv_heads * head_dim and positions.size >= tokens
    kind, (fac, low, high, orig) = (1, llama3) if llama3 is not None else (0, (0.0, 0.0, 0.0, 0))
    _check(lib().oracle_rope(_ptr(q), _ptr(k), _ptr(positions), _dt(q), tokens, q_heads, kv_heads, head_dim,
                             rotary_dim, kind, int(interleaved), ctypes.c_float(theta), ctypes.c_float(fac),
                             ctypes.c_float(low), ctypes.c_float(high), int(orig)))


def qkv_qk_norm_rope_cache_write(qkv, q_out, q_weight, k_weight, positions, k_cache, v_cache, slot_mapping, *, tokens,
                                 q_heads, kv_heads, head_dim, page_size, eps, theta) -> None:
    """CpuOps.QkvQkNormRopeCacheWrite (CpuOps.Fused.cs:37-95): its unfused parts in order. q is copied out of each
    [q | k | v] row into q_out and k, v into scratch; QkNorm of q and k; Rope (full rotary width, default kind, NeoX
    halves) of q and k; CacheWrite of k and v into NHD pools. A cache element type wider than the activations (f32
    pools under bf16 rows) takes the exact widening CpuOps' CopyConvert makes at unit scale."""
    qw, kw = q_heads * head_dim, kv_heads * head_dim
    rows = qkv.reshape(tokens, qw + 2 * kw)
    q_out.reshape(tokens, qw)[:] = rows[:, :qw]
    k = np.ascontiguousarray(rows[:, qw:qw + kw]).reshape(-1)
    v = np.ascontiguousarray(rows[:, qw + kw:]).reshape(-1)
    qk_norm(q_out, k, q_weight, k_weight, tokens=tokens, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, eps=eps)
    rope(q_out, k, positions, tokens=tokens, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, theta=theta)
    if k_cache.dtype != k.dtype:
        assert k.dtype == np.uint16 and k_cache.dtype == np.float32, "only bf16 rows into f32 pools widen exactly"
        k = (k.astype(np.uint32) << 16).view(np.float32)
        v = (v.astype(np.uint32) << 16).view(np.float32)
    cache_write(k, v, k_cache, v_cache, slot_mapping, tokens=tokens, kv_heads=kv_heads, head_dim=head_dim,
                page_size=page_size, bf16=k.dtype == np.uint16)


def state_copy(pool: np.ndarray, pairs: np.ndarray, *, slot_bytes: int) -> None:
    """CpuOps.RecurrentStateCopy: slot pairs[i, 0] -> slot pairs[i, 1] of pool, in pair order."""
    raw = pool.view(np.uint8)
    _check(lib().oracle_state_copy_pairs(_ptr(raw), ctypes.c_int64(raw.size), _ptr(raw), ctypes.c_int64(raw.size),
                                         _ptr(pairs), pairs.size // 2, ctypes.c_int64(slot_bytes), 0))


def state_snapshot(pool: np.ndarray, snapshots: np.ndarray, pairs: np.ndarray, *, slot_bytes: int,
                   restore: bool) -> None:
    """CpuOps.RecurrentStateSnapshot: pairs (slot, snapshot); restore copies snapshot -> slot."""
    p, s = pool.view(np.uint8), snapshots.view(np.uint8)
    src, dst = (s, p) if restore else (p, s)
    _check(lib().oracle_state_copy_pairs(_ptr(src), ctypes.c_int64(src.size), _ptr(dst), ctypes.c_int64(dst.size),
                                         _ptr(pairs), pairs.size // 2, ctypes.c_int64(slot_bytes), int(restore)))


def plan_region(seqs, block_size: int):
    """PlanRegionWriter.Fill over sequences given as dicts with token_start, token_count, position_offset, kv_length
    and blocks. Returns (q_indptr, cu_seqlens, kv_indptr, kv_indices, kv_last_page_len, slot_mapping)."""
    b = len(seqs)
    i32 = lambda xs: np.ascontiguousarray(np.array(xs, dtype=np.int32))
    ts = i32([s["token_start"] for s in seqs])
    tc = i32([s["token_count"] for s in seqs])
    po = i32([s["position_offset"] for s in seqs])
    kl = i32([s["kv_length"] for s in seqs])
    bi = i32(np.concatenate([[0], np.cumsum([len(s["blocks"]) for s in seqs])]))
    blocks = i32(np.concatenate([np.asarray(s["blocks"], dtype=np.int32) for s in seqs]) if b else [])
    tokens = int((ts + tc).max()) if b else 0
    q_indptr = np.zeros(b + 1, np.int32)
    cu = np.zeros(b + 1, np.int32)
    kv_indptr = np.zeros(b + 1, np.int32)
    kv_indices = np.zeros(max(int(bi[-1]), 1), np.int32)
    last = np.zeros(max(b, 1), np.int32)
    slots = np.zeros(max(tokens, 1), np.int64)
    _check(lib().oracle_plan_region(b, _ptr(ts), _ptr(tc), _ptr(po), _ptr(kl), _ptr(bi), _ptr(blocks), block_size,
                                    _ptr(q_indptr), _ptr(cu), _ptr(kv_indptr), _ptr(kv_indices), _ptr(last),
                                    _ptr(slots)))
    return q_indptr, cu, kv_indptr, kv_indices[: int(bi[-1])], last[:b], slots[:tokens]


def host_threads() -> int:
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
