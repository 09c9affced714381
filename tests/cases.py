"""Seeded inputs and comparison rules shared by the parity tests.

Batch shapes follow the reference's GPU harness (kernels/tests/ops-cuda/AttentionCases.cs:83-122: shuffled page pools
with 3 spare pages) and BASELINE.json's configs; GDN inputs follow kernels/tests/hybrid-conformance/GdnCases.cs:135-190
(the fused [tokens, 6144] conv1d output whose column slices are the q, k, v views).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import oracle

# attention and GDN outputs within max-abs 2e-2 AND max-rel 1e-2 (bf16 I/O, fp32 accumulation); GDN
# final state within 1e-3 relative. The relative error of element i is |d_i| / (|ref_i| + max_j |ref_j|): the scaled
# metric the reference's kernel README uses, so that near-zero reference elements do not dominate.
MAX_ABS = 2e-2
MAX_REL = 1e-2
STATE_REL = 1e-3


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return oracle.f32_to_bf16_rne(np.asarray(x, dtype=np.float32))


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return oracle.bf16_to_f64(bits)


def errors(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    assert np.all(np.isfinite(got)), "non-finite output"
    d = np.abs(got - ref)
    denom = np.abs(ref) + (np.abs(ref).max() if ref.size else 0.0)
    rel = d / np.where(denom > 0, denom, 1.0)
    return float(d.max(initial=0.0)), float(rel.max(initial=0.0))


def assert_close(got, ref, max_abs=MAX_ABS, max_rel=MAX_REL, what=""):
    a, r = errors(got, ref)
    assert a <= max_abs and r <= max_rel, f"{what}: max_abs={a:.3e} (tol {max_abs}) max_rel={r:.3e} (tol {max_rel})"
    return a, r


def assert_attention_class(got, ref, v_max, what=""):
    """The reference harness's attention-bf16 class (kernels/tests/ops-cuda/AttentionCases.cs:16 with Compare.cs:14):
    |gpu - ref| <= 2^-8 * max|V| + 2^-7 * |ref| per element."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    allowed = 2.0 ** -8 * v_max + 2.0 ** -7 * np.abs(ref)
    util = np.abs(got - ref) / allowed
    assert util.max(initial=0.0) <= 1.0, f"{what}: attention-bf16 utilisation {util.max():.3f}"
    return float(util.max(initial=0.0))


@dataclass
class PagedBatch:
    """A paged batch on the host: q [tokens, hq, d], pools, tables. bf16 tensors are uint16 bit arrays."""
    q: np.ndarray
    k_cache: np.ndarray
    v_cache: np.ndarray
    q_indptr: np.ndarray
    kv_indptr: np.ndarray
    kv_indices: np.ndarray
    kv_last_page_len: np.ndarray
    kv_lens: list
    q_lens: list
    page_size: int
    hnd: bool
    bf16: bool
    hq: int = 8
    hkv: int = 2
    d: int = 256
    extra: dict = field(default_factory=dict)

    @property
    def batch(self):
        return len(self.kv_lens)

    @property
    def tokens(self):
        return int(self.q_indptr[-1])


def make_paged_batch(rng: np.random.Generator, kv_lens, q_lens, page_size=16, hnd=False, bf16=True, hq=8, hkv=2,
                     d=256, std=1.0, pool_factor=None, spare_pages=3) -> PagedBatch:
    kv_lens = [int(x) for x in kv_lens]
    q_lens = [int(x) for x in q_lens]
    pages = [(kv + page_size - 1) // page_size for kv in kv_lens]
    total = sum(pages)
    pool = int(np.ceil(total * pool_factor)) if pool_factor else total + spare_pages
    perm = rng.permutation(pool).astype(np.int32)
    kv_indices = np.ascontiguousarray(perm[:total])
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    last = np.array([kv - (p - 1) * page_size if p > 0 else 1 for kv, p in zip(kv_lens, pages)], dtype=np.int32)
    tokens = int(q_indptr[-1])
    shape = (pool, hkv, page_size, d) if hnd else (pool, page_size, hkv, d)
    q = (rng.standard_normal((tokens, hq, d), dtype=np.float32) * std)
    k = (rng.standard_normal(shape, dtype=np.float32) * std)
    v = (rng.standard_normal(shape, dtype=np.float32) * std)
    if bf16:
        q, k, v = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    return PagedBatch(q, k, v, q_indptr, kv_indptr, kv_indices, last, kv_lens, q_lens, page_size, hnd, bf16, hq, hkv, d)


def oracle_attention(b: PagedBatch, causal=True, threads=None, window_left=-1, soft_cap=0.0) -> np.ndarray:
    out = np.zeros_like(b.q)
    oracle.paged_attention(b.q, out, b.k_cache, b.v_cache, b.q_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len,
                           soft_cap=soft_cap,
                           batch=b.batch, tokens=b.tokens, q_heads=b.hq, kv_heads=b.hkv, head_dim=b.d,
                           page_size=b.page_size, hnd=b.hnd, causal=causal, bf16=b.bf16, window_left=window_left,
                           threads=threads or oracle.host_threads())
    return out


def values(a: np.ndarray, bf16: bool) -> np.ndarray:
    return bf16_values(a) if bf16 else np.asarray(a, dtype=np.float64)


# ---- GDN ------------------------------------------------------------------------------------------------------------

HEADS, DIM = 16, 128
ROW = HEADS * DIM
FUSED = 3 * ROW


@dataclass
class GdnData:
    fused: np.ndarray  # [tokens, 6144] bf16 bits: q | k | v columns
    g: np.ndarray      # [tokens, 16] f32
    beta: np.ndarray   # [tokens, 16] bf16 bits
    pool: np.ndarray   # [slots, 16, 128, 128] f32
    slots: np.ndarray  # [batch] i32
    cu: np.ndarray     # [batch + 1] i32
    lens: list

    @property
    def tokens(self):
        return int(self.cu[-1])

    @property
    def batch(self):
        return len(self.lens)

    def view(self, which: int) -> np.ndarray:
        """Contiguous copy of the q (0), k (1) or v (2) column slice."""
        return np.ascontiguousarray(self.fused[:, which * ROW:(which + 1) * ROW])


def make_gdn(rng: np.random.Generator, lens, pool_slots, slots=None, decay=None, state_std=0.1, qk_normal=True,
             baseline_style=False) -> GdnData:
    """baseline_style: BASELINE.json config 4 distributions -- beta = sigmoid(N(0,1)), g = -softplus(N(0,1)),
    S0 ~ N(0, 0.01) (0.01 taken as the standard deviation); otherwise the reference harness's (g = -U(0, decay),
    beta = U(0, 1))."""
    tokens = int(sum(lens))
    fused = bf16_bits(rng.standard_normal((tokens, FUSED), dtype=np.float32))
    if baseline_style:
        g = (-np.logaddexp(0.0, rng.standard_normal((tokens, HEADS)))).astype(np.float32)
        beta = bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal((tokens, HEADS)))))
        pool = (rng.standard_normal((pool_slots, HEADS, DIM, DIM), dtype=np.float32) * 0.01).astype(np.float32)
    else:
        g = (-rng.random((tokens, HEADS)) * (decay if decay is not None else 0.2)).astype(np.float32)
        beta = bf16_bits(rng.random((tokens, HEADS)).astype(np.float32))
        pool = (rng.standard_normal((pool_slots, HEADS, DIM, DIM), dtype=np.float32) * state_std).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    if slots is None:
        slots = [(i * 5 + 3) % pool_slots for i in range(len(lens))]
    return GdnData(fused, np.ascontiguousarray(g), np.ascontiguousarray(beta), np.ascontiguousarray(pool),
                   np.array(slots, dtype=np.int32), cu, list(lens))


def oracle_gdn(d: GdnData, use_initial_state=True, threads=None):
    """Returns (output bits, pool after). Runs CpuOps.GatedDeltaRule on the strided views of the fused buffer."""
    out = np.zeros((d.tokens, HEADS, DIM), dtype=np.uint16)
    pool = d.pool.copy()
    q, k, v = d.view(0), d.view(1), d.view(2)
    oracle.gated_delta_rule(q, k, v, d.g, d.beta, out, pool, d.slots, d.cu, batch=d.batch, tokens=d.tokens,
                            k_heads=HEADS, v_heads=HEADS, k_dim=DIM, v_dim=DIM, use_initial_state=use_initial_state,
                            l2_norm_qk=True, scale=0.0, bf16=True, beta_bf16=True,
                            threads=threads or oracle.host_threads())
    return out, pool
