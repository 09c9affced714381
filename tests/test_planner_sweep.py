"""The attention planner on the host across many shapes, without a GPU: the workspace query runs the whole plan
(decode ranges, prefill items and pieces, the mixed-step overlap choice, merges) on the host tables. Every admitted
shape must be planned without a crash, quickly, into a workspace of plausible size; ill-formed tables are refused.
CPU only (the plan's copy to the device is the only GPU step, and the query does not make it)."""
import ctypes as C
import time

import numpy as np
import pytest

import roost_amd
from roost_amd import abi


def _fake(n, dtype):
    s = abi.DeviceSpan()
    s.address = 0x10000
    s.length = n
    s.dtype = dtype
    return s


def _params(kv_lens, q_lens, page_size, head_dim, q_heads, kv_heads, hnd, window, prefill):
    kv_lens = np.asarray(kv_lens, np.int64)
    q_lens = np.asarray(q_lens, np.int64)
    pages = (kv_lens + page_size - 1) // page_size
    qi = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ki = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    last = np.where(pages > 0, kv_lens - (pages - 1) * page_size, 1).astype(np.int32)
    p = abi.new(abi.PagedAttentionParams)
    p.mode = abi.ATTENTION_PREFILL if prefill else abi.ATTENTION_DECODE
    p.batch, p.tokens = len(kv_lens), int(qi[-1])
    p.q_heads, p.kv_heads, p.head_dim, p.page_size = q_heads, kv_heads, head_dim, page_size
    p.kv_layout = abi.LAYOUT_PAGED_HND if hnd else abi.LAYOUT_PAGED_NHD
    p.window_left = window
    for name in ("q", "output", "k_cache", "v_cache"):
        setattr(p, name, _fake(1 << 40, abi.DTYPE_BF16))
    for name in ("q_indptr", "kv_indptr", "kv_last_page_len", "kv_indices"):
        setattr(p, name, _fake(1 << 30, abi.DTYPE_I32))
    keep = (qi, ki, last)
    p.q_indptr_host, p.kv_indptr_host, p.kv_last_page_len_host = (a.ctypes.data for a in keep)
    return p, keep


def _shapes():
    rng = np.random.default_rng(101)
    out = []
    for i in range(160):
        prefill = i % 2 == 1
        batch = int(rng.choice([1, 2, 7, 48, 64, 300, 2048]))
        page_size = int(rng.choice([16, 16, 32, 64, 8, 7]))
        head_dim = int(rng.choice([64, 128, 256]))
        group = int(rng.choice([4, 8, 16, 32]))
        kv_heads = int(rng.choice([1, 2, 4]))
        if prefill and head_dim != 256 and (page_size % 16 or page_size & (page_size - 1)):
            page_size = 16  # the refused combination is covered elsewhere
        kv = rng.integers(0, int(rng.choice([17, 600, 9000, 70000])), size=batch)
        if prefill:
            q = np.minimum(kv, rng.choice([1, 1, 64, 512, 3000], size=batch))
            q = np.where(kv == 0, 0, np.maximum(q, 0))
        else:
            kv = np.maximum(kv, 0)
            q = np.ones(batch, np.int64)
        window = int(rng.choice([-1, -1, 1, 100, 4096]))
        out.append((kv, q, page_size, head_dim, group * kv_heads, kv_heads, bool(rng.integers(2)), window, prefill))
    # extremes: one very long sequence, many decode rows, a mixed step with huge contexts
    out.append(([2_000_000], [1], 16, 256, 8, 2, False, -1, False))
    out.append(([300_000], [300_000], 16, 128, 8, 2, False, -1, True))
    out.append(([5] * 100_000, [1] * 100_000, 16, 256, 8, 2, False, -1, False))
    out.append((list(range(1024, 1024 + 48 * 300, 300)) + [4608, 4608], [1] * 48 + [512, 512], 16, 256, 8, 2, False,
                -1, True))
    return out


@pytest.mark.parametrize("case", range(len(_shapes())))
def test_attention_planner_on_the_host(kernels, case):
    kv, q, ps, d, hq, hkv, hnd, window, prefill = _shapes()[case]
    p, keep = _params(kv, q, ps, d, hq, hkv, hnd, window, prefill)
    e = kernels.entry(roost_amd.ATTENTION_VARIANT)
    ctx = kernels.create_context(0)
    sizes = abi.new(abi.WorkspaceSizes)
    t0 = time.perf_counter()
    status = e.workspace(ctx, C.addressof(p), C.addressof(sizes))
    elapsed = time.perf_counter() - t0
    kernels.destroy_context(ctx)
    assert status == abi.OK, kernels.last_error()
    q = np.asarray(q)
    tokens = int(q.sum())
    # Plausible sizes: the host tables are within the device region, and the partials are bounded by the planner's
    # own limits -- tile pieces at most the items plus two per CU (256 rows each: 64 tokens x 4 query heads, bf16 with
    # a (max, sum) pair), decode pieces at most the decode rows plus two ranges per CU and head block (fp32 rows).
    vheads = hq // 4
    multi = q[q > 1] if prefill else q[:0]
    items = int(np.sum((multi + 63) // 64)) * vheads
    dec_rows = int(np.sum(q == 1)) if prefill else tokens
    bound = (64 * (len(kv) + tokens + items + 4096) + (items + 2 * 256) * 256 * (2 * d + 8)
             + (dec_rows + 2 * 256 * vheads) * hq * (d + 2) * 4)
    assert sizes.pinned_host_bytes <= sizes.device_bytes
    assert sizes.device_bytes <= bound, (sizes.device_bytes, bound)
    assert elapsed < 2.0, f"planning took {elapsed:.2f} s"
    del keep
