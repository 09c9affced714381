"""Whole worker steps on the GPU through the C ABI, each call checked against the CpuOps oracle.

- one step of a 3:1 GDN:attention layer group. The step's tables come from the plan-region rule
  (src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64, restated in oracle.plan_region): 48 decode sequences
  (contexts U(1024, 16384)) and 2 chunks of 512 tokens on 4096-token prefixes. CacheWrite appends the step's 1,072 new
  K/V rows at their slots (bit-exact), one prefill-mode PagedAttention call reads them back, and three GatedDeltaRule
  calls on the recurrent variant (the one the worker binds, CudaOps.cs:28) update 50 sequences each in one shared
  150-slot state pool (outputs within 2e-2 / 1e-2, states within 1e-3).
- BASELINE config 3 with its append: the chunks' new K/V rows are written into freshly allocated random pages by
  CacheWrite before the attention call reads them.
"""
import numpy as np
import pytest

import cases
import oracle
import roost_amd
from cases import HEADS
from roost_amd import abi
from test_attention_gpu import Dev, from_dev, to_dev, torch_reference
from test_gdn_gpu import DevGdn

pytestmark = pytest.mark.gpu


def _region(rng, kv_lens, q_lens, page_size=16, pool_factor=1.25):
    """Disjoint random page lists from a pool of pool_factor x the pages the step needs, and the step's tables by the
    plan-region rule."""
    pages = [(kv + page_size - 1) // page_size for kv in kv_lens]
    pool = int(np.ceil(sum(pages) * pool_factor))
    perm = rng.permutation(pool).astype(np.int32)
    seqs, start, used = [], 0, 0
    for kv, n, p in zip(kv_lens, q_lens, pages):
        seqs.append(dict(token_start=start, token_count=int(n), position_offset=int(kv - n), kv_length=int(kv),
                         blocks=perm[used:used + p]))
        start += int(n)
        used += p
    return pool, oracle.plan_region(seqs, page_size)


def _sequence(b: cases.PagedBatch, s: int) -> cases.PagedBatch:
    """Sequence s of a batch as a batch of its own over the same pools."""
    n = int(b.q_indptr[s + 1] - b.q_indptr[s])
    return cases.PagedBatch(b.q[b.q_indptr[s]:b.q_indptr[s + 1]].copy(), b.k_cache, b.v_cache,
                            np.array([0, n], np.int32), np.array([0, b.kv_indptr[s + 1] - b.kv_indptr[s]], np.int32),
                            b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]].copy(), b.kv_last_page_len[s:s + 1].copy(),
                            [int(b.kv_lens[s])], [n], b.page_size, b.hnd, True, b.hq, b.hkv, b.d)


def _append(session, rng, b: cases.PagedBatch, slots: np.ndarray):
    """Replaces the rows at `slots` in the device pools with garbage, then CacheWrites the batch's true rows there.
    Returns the device batch; its pools must equal b's bit for bit."""
    tokens, hkv, d = slots.size, b.hkv, b.d
    ps = b.page_size
    page, off = slots // ps, slots % ps
    k_new = np.ascontiguousarray(b.k_cache[page, off])  # [tokens, hkv, d]
    v_new = np.ascontiguousarray(b.v_cache[page, off])
    stale_k, stale_v = b.k_cache.copy(), b.v_cache.copy()
    stale_k[page, off] = rng.integers(0, 65536, size=(tokens, hkv, d), dtype=np.uint16)
    stale_v[page, off] = 0xABAB
    stale = cases.PagedBatch(b.q, stale_k, stale_v, b.q_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len,
                             b.kv_lens, b.q_lens, b.page_size, b.hnd, True, b.hq, b.hkv, b.d)
    dev = Dev(stale)
    roost_amd.cache_write(session, to_dev(k_new, True), to_dev(v_new, True), dev.k, dev.v, to_dev(slots),
                          kv_heads=hkv, head_dim=d, page_size=ps, kv_layout=abi.LAYOUT_PAGED_NHD)
    # CpuOps.CacheWrite on the host copy gives the same pools.
    want_k, want_v = stale_k.copy(), stale_v.copy()
    oracle.cache_write(k_new, v_new, want_k, want_v, slots, tokens=tokens, kv_heads=hkv, head_dim=d, page_size=ps,
                       bf16=True)
    got_k, got_v = from_dev(dev.k, True), from_dev(dev.v, True)
    assert np.array_equal(want_k, b.k_cache) and np.array_equal(want_v, b.v_cache)
    assert np.array_equal(got_k, want_k), "CacheWrite K pool differs from CpuOps"
    assert np.array_equal(got_v, want_v), "CacheWrite V pool differs from CpuOps"
    dev.b = b
    return dev


def _attention(session, dev: Dev):
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    session.launch(entry, dev.params(), key=("step", dev.b.batch, dev.b.tokens))
    return dev.result()


def test_config3_append_then_prefill(session):
    rng = np.random.default_rng(33)
    n = rng.integers(256, 2049, size=8)
    pre = rng.integers(0, 6145, size=8)
    kv = n + pre
    pool, (q_indptr, _, kv_indptr, kv_indices, last, slots) = _region(rng, kv, n)
    b = cases.make_paged_batch(rng, kv, n, std=0.5, pool_factor=1.25)
    b.kv_indices, b.kv_indptr, b.kv_last_page_len = kv_indices, kv_indptr, last
    assert np.array_equal(b.q_indptr, q_indptr) and b.k_cache.shape[0] >= pool
    dev = _append(session, rng, b, slots)
    got = _attention(session, dev)
    cases.assert_close(got, torch_reference(b), what="config 3 after append vs fp32 torch")
    s = int(np.argmin(kv))
    cases.assert_close(got[b.q_indptr[s]:b.q_indptr[s + 1]],
                       cases.values(cases.oracle_attention(_sequence(b, s)), True), what=f"config 3 seq {s} vs CpuOps")


def test_config5_worker_step(session):
    import torch

    rng = np.random.default_rng(55)
    kv = np.concatenate([rng.integers(1024, 16385, size=48), [4608, 4608]])
    n = np.concatenate([np.ones(48, np.int64), [512, 512]])
    pool, (q_indptr, cu, kv_indptr, kv_indices, last, slots) = _region(rng, kv, n)
    b = cases.make_paged_batch(rng, kv, n, std=0.5, pool_factor=1.25)
    b.kv_indices, b.kv_indptr, b.kv_last_page_len = kv_indices, kv_indptr, last
    assert slots.size == 1072 and b.k_cache.shape[0] >= pool

    # 1. CacheWrite of the step's new rows (bit-exact), then the attention call that reads them.
    dev = _append(session, rng, b, slots)
    got = _attention(session, dev)
    for s in (int(np.argmin(kv[:48])), int(np.argmax(kv[:48])), 48, 49):
        cases.assert_close(got[b.q_indptr[s]:b.q_indptr[s + 1]],
                           cases.values(cases.oracle_attention(_sequence(b, s)), True),
                           what=f"config 5 attention seq {s} vs CpuOps")
    del dev

    # 2. Three GDN layers on the recurrent variant, layer L's sequences in slots 50 L .. 50 L + 49 of one pool.
    lens = [int(x) for x in n]
    assert np.array_equal(cu, np.concatenate([[0], np.cumsum(lens)]))
    shared = (rng.standard_normal((150, HEADS, 128, 128), dtype=np.float32) * 0.01).astype(np.float32)
    pool_dev = to_dev(shared)
    want_pool = shared.copy()
    for layer in range(3):
        d = cases.make_gdn(rng, lens, 150, slots=list(range(50 * layer, 50 * layer + 50)), baseline_style=True)
        d.pool = want_pool
        want_o, want_pool = cases.oracle_gdn(d)
        g = DevGdn(d)
        g.pool = pool_dev  # the step's shared pool, carried from layer to layer
        session.launch(session.lib.entry(roost_amd.RECURRENT_VARIANT), g.params(), key=("step gdn", layer))
        got_o = from_dev(g.out, True)[: d.tokens]
        cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o), what=f"config 5 GDN layer {layer}")
    torch.cuda.synchronize()
    got_pool = from_dev(pool_dev)
    for s in range(150):
        cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"config 5 slot {s}")
