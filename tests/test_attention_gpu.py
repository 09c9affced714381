"""PagedAttention on the GPU through the C ABI vs the CpuOps oracle (reference harness:
kernels/tests/ops-cuda/AttentionCases.cs:29-288). Tolerances: BASELINE.json's max-abs 2e-2 and max-rel 1e-2 for bf16
I/O, plus the reference harness's attention-bf16 class; 1e-5 for the fp32 decode of config 1."""
import ctypes as C
import zlib

import numpy as np
import pytest

import cases
import roost_amd
from roost_amd import abi

pytestmark = pytest.mark.gpu


def torch():
    import torch as t

    return t


def to_dev(a: np.ndarray, bf16=False):
    t = torch()
    x = t.from_numpy(np.ascontiguousarray(a))
    if bf16:
        x = x.view(t.bfloat16)
    return x.cuda()


def from_dev(x, bf16=False):
    t = torch()
    t.cuda.synchronize()
    if bf16:
        return x.view(t.int16).cpu().numpy().view(np.uint16)
    return x.cpu().numpy()


class Dev:
    """A PagedBatch on the device plus its params."""

    def __init__(self, b: cases.PagedBatch, causal=True, with_lse=False, window_left=-1, soft_cap=0.0):
        self.b = b
        self.q = to_dev(b.q, b.bf16)
        self.k = to_dev(b.k_cache, b.bf16)
        self.v = to_dev(b.v_cache, b.bf16)
        self.q_indptr = to_dev(b.q_indptr)
        self.kv_indptr = to_dev(b.kv_indptr)
        self.kv_indices = to_dev(b.kv_indices if b.kv_indices.size else np.zeros(1, np.int32))
        self.last = to_dev(b.kv_last_page_len)
        self.out = torch().full_like(self.q, float("nan"))
        self.lse = torch().zeros((b.tokens, b.hq), dtype=torch().float32, device="cuda") if with_lse else None
        self.causal = causal
        self.window_left = window_left
        self.soft_cap = soft_cap

    def params(self, host=True, **over):
        b = self.b
        kw = dict(q_indptr_host=b.q_indptr if host else None, kv_indptr_host=b.kv_indptr if host else None,
                  kv_last_page_len_host=b.kv_last_page_len if host else None, batch=b.batch, q_heads=b.hq,
                  kv_heads=b.hkv, head_dim=b.d, page_size=b.page_size,
                  kv_layout=abi.LAYOUT_PAGED_HND if b.hnd else abi.LAYOUT_PAGED_NHD, causal=self.causal, lse=self.lse,
                  window_left=self.window_left, soft_cap=self.soft_cap)
        kw.update(over)
        return roost_amd.paged_attention_params(self.q, self.out, self.k, self.v, self.q_indptr, self.kv_indptr,
                                                self.kv_indices, self.last, **kw)

    def result(self):
        return cases.values(from_dev(self.out, self.b.bf16), self.b.bf16)


def run_case(session, b: cases.PagedBatch, causal=True, check_nohost=True, check_determinism=True, window_left=-1):
    d = Dev(b, causal, window_left=window_left)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    p = d.params()
    # Run before plan: NOT_PLANNED (a fresh, zeroed plan record).
    sizes = session.workspace_sizes(entry, p)
    ws = abi.new(abi.Workspace)
    plan_buf = C.create_string_buffer(max(int(sizes.plan_bytes), 1))
    ws.plan, ws.plan_bytes = C.addressof(plan_buf), sizes.plan_bytes
    assert session.run_raw(entry, p, ws) == abi.NOT_PLANNED
    session.launch(entry, p, key=("case", b.batch, b.tokens))
    got = from_dev(d.out, b.bf16)
    if check_nohost:
        # run() never reads the host tables: NULL host pointers give the same bits (AttentionCases.cs:216-224).
        d.out.fill_(float("nan"))
        session.run(entry, d.params(host=False), session._ws[(entry.variant_id, ("case", b.batch, b.tokens))][3])
        assert np.array_equal(from_dev(d.out, b.bf16), got)
    if check_determinism:
        d.out.fill_(float("nan"))
        session.launch(entry, p, key=("case", b.batch, b.tokens))
        assert np.array_equal(from_dev(d.out, b.bf16), got), "second run is not bit-identical"
    return cases.values(got, b.bf16)


def torch_reference(b: cases.PagedBatch, causal=True) -> np.ndarray:
    """The same attention in float32 torch on the GPU over de-paged K/V (NHD bf16 pools): the whole-batch check for
    shapes too large for the double-precision CpuOps oracle."""
    t = torch()
    qv = t.from_numpy(cases.values(b.q, True).astype(np.float32)).cuda()
    kc = t.from_numpy(cases.values(b.k_cache, True).astype(np.float32)).cuda()
    vc = t.from_numpy(cases.values(b.v_cache, True).astype(np.float32)).cuda()
    ref = np.zeros(b.q.shape, np.float64)
    group = b.hq // b.hkv
    for s in range(b.batch):
        pages = t.from_numpy(b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]].astype(np.int64)).cuda()
        kl = int(b.kv_lens[s])
        k = kc[pages].reshape(-1, b.hkv, b.d)[:kl]
        v = vc[pages].reshape(-1, b.hkv, b.d)[:kl]
        q = qv[b.q_indptr[s]:b.q_indptr[s + 1]]
        qpos = t.arange(kl - q.shape[0], kl, device="cuda")
        mask = t.arange(kl, device="cuda")[None, :] <= qpos[:, None]
        for h in range(b.hq):
            sc = (q[:, h, :] @ k[:, h // group, :].T) / float(np.sqrt(b.d))
            if causal:
                sc = sc.masked_fill(~mask, float("-inf"))
            ref[b.q_indptr[s]:b.q_indptr[s + 1], h] = (t.softmax(sc, dim=-1) @ v[:, h // group, :]).cpu().numpy()
    return ref


def check_against_oracle(got, b, causal=True, window_left=-1):
    ref = cases.values(cases.oracle_attention(b, causal, window_left=window_left), b.bf16)
    a, r = cases.assert_close(got, ref, what="attention")
    if b.bf16:
        cases.assert_attention_class(got, ref, float(np.abs(cases.values(b.v_cache, True)).max()), what="attention")
    return a, r


DECODE_CASES = [
    ("mixed4 NHD ps16", [5, 37, 130, 16], 16, False),
    ("mixed4 HND ps16", [5, 37, 130, 16], 16, True),
    ("mixed4 NHD ps32", [5, 37, 130, 16], 32, False),
    ("mixed4 HND ps64", [5, 37, 130, 16], 64, True),
    ("single-token-history", [1], 16, False),
    ("page-multiples", [16, 32, 48, 64], 16, False),
    ("single-6000 split", [6000], 16, False),
    ("mixed8", [900, 17, 1, 2048, 333, 64, 1024, 777], 16, False),
    ("mixed8 HND ps64", [900, 17, 1, 2048, 333, 64, 1024, 777], 64, True),
    ("odd page size 7", [5, 37, 130, 1000], 7, False),
]


@pytest.mark.parametrize("name,kv_lens,ps,hnd", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_decode_bf16_matches_cpuops(session, name, kv_lens, ps, hnd):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, kv_lens, [1] * len(kv_lens), page_size=ps, hnd=hnd)
    got = run_case(session, b)
    check_against_oracle(got, b)


def test_decode_batch64_short(session):
    rng = np.random.default_rng(64)
    kv = rng.integers(1, 301, size=64)
    b = cases.make_paged_batch(rng, kv, [1] * 64)
    check_against_oracle(run_case(session, b), b)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_head_dims_bf16(session, d):
    rng = np.random.default_rng(d)
    b = cases.make_paged_batch(rng, [3, 700, 40], [1, 1, 1], d=d)
    check_against_oracle(run_case(session, b), b)


def test_config1_fp32_decode_with_kv_append(session):
    """fp32, hd 64, 8q/2kv, B=4, ctx ~ U(17, 300), page 16, randomly permuted block table into a
    64-page pool, Q/K/V ~ N(0, 1), scale 1/8; the new token's K/V is appended at its slot-mapped position first."""
    import oracle

    t = torch()
    rng = np.random.default_rng(1)
    kv_lens = rng.integers(17, 301, size=4)
    b = cases.make_paged_batch(rng, kv_lens, [1] * 4, page_size=16, bf16=False, d=64, pool_factor=None,
                               spare_pages=64 - sum((int(k) + 15) // 16 for k in kv_lens))
    assert b.k_cache.shape[0] == 64
    # Slot mapping of the new token (position kvLen - 1) through the plan-region rule.
    seqs, start = [], 0
    for i, kv in enumerate(b.kv_lens):
        blocks = b.kv_indices[b.kv_indptr[i]:b.kv_indptr[i + 1]]
        seqs.append(dict(token_start=i, token_count=1, position_offset=kv - 1, kv_length=kv, blocks=blocks))
    _, _, _, _, _, slots = oracle.plan_region(seqs, 16)
    new_k = rng.standard_normal((4, 2, 64), dtype=np.float32)
    new_v = rng.standard_normal((4, 2, 64), dtype=np.float32)
    k_ref, v_ref = b.k_cache.copy(), b.v_cache.copy()
    oracle.cache_write(new_k, new_v, k_ref, v_ref, slots, tokens=4, kv_heads=2, head_dim=64, page_size=16)
    d = Dev(b)
    roost_amd.cache_write(session, to_dev(new_k), to_dev(new_v), d.k, d.v, to_dev(slots), kv_heads=2, head_dim=64,
                          page_size=16)
    assert np.array_equal(from_dev(d.k), k_ref) and np.array_equal(from_dev(d.v), v_ref), "KV append not bit-exact"
    b.k_cache, b.v_cache = k_ref, v_ref
    session.launch(session.lib.entry(roost_amd.ATTENTION_VARIANT), d.params(sm_scale=0.125), key="cfg1")
    got = d.result()
    out = np.zeros_like(b.q)
    oracle.paged_attention(b.q, out, k_ref, v_ref, b.q_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, batch=4,
                           tokens=4, q_heads=8, kv_heads=2, head_dim=64, page_size=16, scale=0.125)
    cases.assert_close(got, out, max_abs=1e-5, max_rel=1e-5, what="config 1 fp32 decode")


def test_config2_decode_full_size(session):
    """BASELINE config 2 at full size: B=64, ctx ~ U(512, 8192), hd 256, bf16, 0.5*N(0,1), pool 1.25x tokens."""
    rng = np.random.default_rng(2)
    kv = rng.integers(512, 8193, size=64)
    b = cases.make_paged_batch(rng, kv, [1] * 64, std=0.5, pool_factor=1.25)
    got = run_case(session, b, check_nohost=False)
    check_against_oracle(got, b)


def test_decode_row_alone_equals_row_in_batch_within_tolerance(session):
    """The decode plan deals the batch's keys out evenly over the workgroups, so how a sequence is split depends on the
    rest of the batch: the variant is DETERMINISTIC (identical batch -> identical bits, checked in run_case) but not
    BATCH_INVARIANT, like the reference's FlashInfer variant. A row computed alone and inside a batch agree to the
    parity tolerance."""
    rng = np.random.default_rng(7)
    b = cases.make_paged_batch(rng, [3000, 17, 900], [1, 1, 1])
    many = run_case(session, b, check_nohost=False, check_determinism=False)
    one = cases.PagedBatch(b.q[:1].copy(), b.k_cache, b.v_cache, np.array([0, 1], np.int32),
                           b.kv_indptr[:2].copy(), b.kv_indices[:b.kv_indptr[1]].copy(), b.kv_last_page_len[:1].copy(),
                           b.kv_lens[:1], [1], b.page_size, b.hnd, b.bf16)
    alone = run_case(session, one, check_nohost=False, check_determinism=False)
    cases.assert_close(alone, many[:1], max_abs=2e-2, max_rel=1e-2, what="alone vs in batch")
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    assert entry.flags & abi.FLAG_DETERMINISTIC and not entry.flags & abi.FLAG_BATCH_INVARIANT


def test_decode_lse_is_base2_logsumexp(session):
    rng = np.random.default_rng(11)
    b = cases.make_paged_batch(rng, [700, 33], [1, 1])
    d = Dev(b, with_lse=True)
    session.launch(session.lib.entry(roost_amd.ATTENTION_VARIANT), d.params(), key="lse")
    lse = from_dev(d.lse)
    qv = cases.values(b.q, True)
    kv = cases.values(b.k_cache, True)
    for s in range(2):
        pages = b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]]
        keys = kv[pages].reshape(-1, 2, 256)[: b.kv_lens[s]]
        for h in range(8):
            sc = keys[:, h // 4, :] @ qv[s, h] / 16.0
            want = np.log2(np.exp(sc - sc.max()).sum()) + sc.max() / np.log(2)
            assert abs(lse[s, h] - want) < 1e-3


def lse_reference(b: cases.PagedBatch, causal=True, window_left=-1) -> np.ndarray:
    """[tokens, hq] base-2 log-sum-exp of each query row's visible scaled scores, in float64 from the de-paged
    K (NaN for a row that sees no key). The library's convention for the optional lse output (FlashInfer's): log2 of
    sum_j exp(s_j) with s_j = q.k_j / sqrt(d)."""
    qv = cases.values(b.q, b.bf16).astype(np.float64)
    kc = cases.values(b.k_cache, b.bf16).astype(np.float64)
    out = np.full((b.tokens, b.hq), np.nan)
    group = b.hq // b.hkv
    for s in range(b.batch):
        pages = b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]]
        kl = int(b.kv_lens[s])
        if b.hnd:
            keys = kc[pages].transpose(0, 2, 1, 3).reshape(-1, b.hkv, b.d)[:kl]
        else:
            keys = kc[pages].reshape(-1, b.hkv, b.d)[:kl]
        q0, q1 = int(b.q_indptr[s]), int(b.q_indptr[s + 1])
        for i in range(q1 - q0):
            pos = kl - (q1 - q0) + i
            hi = pos + 1 if causal or q1 - q0 == 1 else kl
            lo = max(0, pos - window_left) if window_left >= 0 else 0
            if hi <= lo:
                continue
            for h in range(b.hq):
                sc = keys[lo:hi, h // group, :] @ qv[q0 + i, h] / np.sqrt(b.d)
                m = sc.max()
                out[q0 + i, h] = (m + np.log(np.exp(sc - m).sum())) / np.log(2.0)
    return out


LSE_PREFILL_CASES = [
    # tile kernel: a 64-token chunk split into many pieces (one-token merge blocks) and a 256-token chunk in two
    # pieces (the 8-token merge form), in one call
    ("tile split, both merge forms", [(64, 12064), (256, 1156)], 16, False, True, -1, 256, True),
    ("tile hd128 HND window", [(300, 2000), (17, 17)], 32, True, True, 200, 128, True),
    ("tile non-causal", [(40, 700)], 16, False, False, -1, 256, True),
    ("general kernel ps8", [(100, 300), (5, 40)], 8, False, True, -1, 256, True),
    ("mixed step: decode rows beside chunks", [(1, 900), (200, 1200), (1, 3000), (1, 17)], 16, False, True, -1, 256,
     True),
    ("f32 prefill rows, split", [(6, 9000), (37, 300)], 16, False, True, -1, 256, False),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window,d,bf16", LSE_PREFILL_CASES,
                         ids=[c[0] for c in LSE_PREFILL_CASES])
def test_prefill_lse_is_base2_logsumexp(session, name, seqs, ps, hnd, causal, window, d, bf16):
    """The optional lse output of prefill calls (roost_kernels.h: PagedAttention's lse span) on every kernel that writes
    it: the tile kernel and both merge forms, the general kernel, the decode rows of a mixed call and f32 prefill
    rows, against float64 log-sum-exp. Bar: 2e-3 absolute (fp32 scores and sums over up to 12k keys)."""
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=d, bf16=bf16)
    dv = Dev(b, causal=causal, with_lse=True, window_left=window)
    dv.lse.fill_(float("nan"))
    session.launch(session.lib.entry(roost_amd.ATTENTION_VARIANT), dv.params(), key=("lse", name))
    got = from_dev(dv.lse)
    want = lse_reference(b, causal, window)
    seen = ~np.isnan(want)
    assert seen.any() and np.isfinite(got[seen]).all(), name
    err = np.abs(got[seen] - want[seen]).max()
    assert err < 2e-3, f"{name}: lse off by {err}"
    # the output rows are unchanged by asking for lse
    check_against_oracle(dv.result(), b, causal=causal, window_left=window) if bf16 else None


def test_decode_zero_length_sequence_outputs_zeros(session):
    rng = np.random.default_rng(5)
    b = cases.make_paged_batch(rng, [40, 0, 17], [1, 1, 1])
    got = run_case(session, b, causal=False, check_nohost=False)
    assert np.all(got[1] == 0)
    check_against_oracle(got, b, causal=False)


PREFILL_CASES = [
    ("one-token", [(1, 1)], 16, False, True),
    ("fresh-100", [(100, 100)], 16, False, True),
    ("fresh-100 HND", [(100, 100)], 16, True, True),
    ("fresh-700 ps64", [(700, 700)], 64, False, True),
    ("fresh-1024", [(1024, 1024)], 16, False, True),
    ("chunk-128-of-1000", [(128, 1000)], 16, False, True),
    ("chunk-128-of-1000 HND ps32", [(128, 1000)], 32, True, True),
    ("multi-seq", [(17, 17), (64, 300), (1, 50), (200, 200)], 16, False, True),
    ("non-causal-32-of-200", [(32, 200)], 16, False, False),
    ("partial-last-page", [(33, 33), (5, 21)], 16, False, True),
    # page sizes that are not multiples of 16 take the general (register-staged) prefill kernel
    ("chunk-100-of-300 ps8", [(100, 300)], 8, False, True),
    ("fresh-40 ps1 HND", [(40, 40)], 1, True, True),
    # a long causal chunk: its key range is cut into pieces that the merge kernel combines
    ("chunk-512-of-4000 split", [(512, 4000), (3, 3)], 16, False, True),
    # merges of two pieces (8 tokens per merge block) and of 3 and 24 pieces (one token per block) in one call
    ("two- and many-piece merges", [(64, 12064), (256, 1156)], 16, False, True),
    # mixed worker steps: the single-token sequences of a prefill call run on the decode kernels
    ("mixed step 6 decode + 2 chunks", [(1, 900), (1, 17), (200, 1200), (1, 3000), (1, 1), (64, 64), (1, 5000),
                                        (1, 333)], 16, False, True),
    ("mixed step HND ps64", [(1, 900), (130, 700), (1, 4000), (2, 2)], 64, True, True),
    ("mixed step ps8", [(1, 900), (100, 300), (1, 45)], 8, False, True),
    ("mixed non-causal with empty row", [(1, 0), (5, 40), (1, 7)], 16, False, False),
    ("all single-token rows in prefill mode", [(1, 50), (1, 3000)], 16, False, True),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_prefill_matches_cpuops(session, name, seqs, ps, hnd, causal):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd)
    got = run_case(session, b, causal=causal)
    check_against_oracle(got, b, causal=causal)


def test_config3_prefill_full_size(session):
    """BASELINE config 3 at full size (8 sequences, chunk U(256, 2048) onto prefix U(0, 6144), causal): the whole batch
    against a float32 torch reference of the same math, and two sampled sequences against the CpuOps oracle."""
    t = torch()
    rng = np.random.default_rng(3)
    n = rng.integers(256, 2049, size=8)
    pre = rng.integers(0, 6145, size=8)
    b = cases.make_paged_batch(rng, n + pre, n, std=0.5, pool_factor=1.25)
    got = run_case(session, b, check_nohost=False, check_determinism=False)
    ref = torch_reference(b)
    cases.assert_close(got, ref, what="config 3 vs fp32 torch")
    for s in (int(np.argmin(n + pre)), 3):
        one = cases.PagedBatch(b.q[b.q_indptr[s]:b.q_indptr[s + 1]].copy(), b.k_cache, b.v_cache,
                               np.array([0, n[s]], np.int32), np.array([0, b.kv_indptr[s + 1] - b.kv_indptr[s]], np.int32),
                               b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]].copy(), b.kv_last_page_len[s:s + 1].copy(),
                               [int(b.kv_lens[s])], [int(n[s])], 16, False, True)
        ref1 = cases.values(cases.oracle_attention(one), True)
        cases.assert_close(got[b.q_indptr[s]:b.q_indptr[s + 1]], ref1, what=f"config 3 seq {s} vs CpuOps")


def test_config5_mixed_step_attention(session):
    """BASELINE config 5's attention call: 48 decode rows (ctx U(1024, 16384)) and 2 chunks of 512 on 4096-token
    prefixes in one prefill-mode call, as the worker issues a mixed step. The whole batch against a float32 torch
    reference of the same math; three sampled sequences (two decode rows and one chunk) against the CpuOps oracle."""
    t = torch()
    rng = np.random.default_rng(5)
    kv = np.concatenate([rng.integers(1024, 16385, size=48), [4608, 4608]])
    n = np.concatenate([np.ones(48, np.int64), [512, 512]])
    b = cases.make_paged_batch(rng, kv, n, std=0.5, pool_factor=1.25)
    got = run_case(session, b, check_nohost=False, check_determinism=True)
    ref = torch_reference(b)
    cases.assert_close(got, ref, what="config 5 attention vs fp32 torch")
    for s in (int(np.argmin(kv[:48])), int(np.argmax(kv[:48])), 49):
        one = cases.PagedBatch(b.q[b.q_indptr[s]:b.q_indptr[s + 1]].copy(), b.k_cache, b.v_cache,
                               np.array([0, n[s]], np.int32), np.array([0, b.kv_indptr[s + 1] - b.kv_indptr[s]], np.int32),
                               b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]].copy(), b.kv_last_page_len[s:s + 1].copy(),
                               [int(b.kv_lens[s])], [int(n[s])], 16, False, True)
        ref1 = cases.values(cases.oracle_attention(one), True)
        cases.assert_close(got[b.q_indptr[s]:b.q_indptr[s + 1]], ref1, what=f"config 5 seq {s} vs CpuOps")


def _plan_overlap(session, key) -> int:
    """The plan record's `overlap` word (its 11th 32-bit field): the decode workgroups a mixed call launches beside its
    tile pieces in one MixedAttentionKernel launch, 0 when the plan runs them one after the other."""
    plan = session._ws[(roost_amd.ATTENTION_VARIANT, key)][2]
    return int(np.frombuffer(bytes(plan)[40:44], np.uint32)[0])


@pytest.mark.parametrize("d,cap", [(128, 0.0), (64, 0.0), (256, 30.0)], ids=["hd128", "hd64", "hd256 soft cap"])
def test_mixed_launch_head_dims_and_soft_cap(session, d, cap):
    """Config 5's shape (48 decode rows of U(1024, 16384) contexts beside two 512-token chunks on 4096-token prefixes)
    at the other head dims and with a logit soft cap: the plan takes the one-launch form (checked in the plan record),
    and the result matches a float32 torch reference of the whole batch (uncapped) and the CpuOps oracle on a short
    and a long decode row and one chunk."""
    rng = np.random.default_rng(50 + d + int(cap))
    kv = np.concatenate([rng.integers(1024, 16385, size=48), [4608, 4608]])
    n = np.concatenate([np.ones(48, np.int64), [512, 512]])
    b = cases.make_paged_batch(rng, kv, n, d=d, std=2.0 if cap else 0.5, pool_factor=1.25)
    dv = Dev(b, soft_cap=cap)
    key = ("mixed-launch", d, cap)
    session.launch(session.lib.entry(roost_amd.ATTENTION_VARIANT), dv.params(), key=key)
    assert _plan_overlap(session, key) > 0, "the plan did not take the one-launch form"
    got = dv.result()
    assert not np.isnan(got).any()
    if not cap:
        cases.assert_close(got, torch_reference(b), what=f"hd{d} mixed launch vs fp32 torch")
    for s in (int(np.argmin(kv[:48])), int(np.argmax(kv[:48])), 49):
        one = cases.PagedBatch(b.q[b.q_indptr[s]:b.q_indptr[s + 1]].copy(), b.k_cache, b.v_cache,
                               np.array([0, n[s]], np.int32), np.array([0, b.kv_indptr[s + 1] - b.kv_indptr[s]], np.int32),
                               b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]].copy(), b.kv_last_page_len[s:s + 1].copy(),
                               [int(b.kv_lens[s])], [int(n[s])], 16, False, True, d=d)
        ref1 = cases.values(cases.oracle_attention(one, soft_cap=cap), True)
        cases.assert_close(got[b.q_indptr[s]:b.q_indptr[s + 1]], ref1, max_abs=(2 if cap else 1) * cases.MAX_ABS,
                           what=f"hd{d} cap {cap} seq {s} vs CpuOps")


def test_prefill_batch_invariance(session):
    rng = np.random.default_rng(9)
    b = cases.make_paged_batch(rng, [333, 500, 129], [333, 100, 129])
    many = run_case(session, b, check_nohost=False, check_determinism=False)
    one = cases.PagedBatch(b.q[:333].copy(), b.k_cache, b.v_cache, np.array([0, 333], np.int32),
                           b.kv_indptr[:2].copy(), b.kv_indices[:b.kv_indptr[1]].copy(), b.kv_last_page_len[:1].copy(),
                           b.kv_lens[:1], [333], 16, False, True)
    alone = run_case(session, one, check_nohost=False, check_determinism=False)
    assert np.array_equal(alone, many[:333])


def test_rejections(session):
    """Typed refusals before any launch (reference AttentionCases.cs:234-288)."""
    rng = np.random.default_rng(4)
    b = cases.make_paged_batch(rng, [40, 17], [1, 1])
    d = Dev(b)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    good = d.params()
    session.launch(entry, good, key="rej")
    ws = session._ws[(entry.variant_id, "rej")][3]

    def status(**over):
        return session.run_raw(entry, d.params(**over), ws)

    assert status(head_dim=96) == abi.UNSUPPORTED
    assert status(q_heads=12) == abi.UNSUPPORTED  # a group of 6 (4, 8, 16 and 32 are built)
    assert status(window_left=0) == abi.INVALID_ARGUMENT  # CpuOps refuses a window of 0; -1 means none
    assert status(soft_cap=float("inf")) == abi.INVALID_ARGUMENT
    p = d.params()
    p.tokens = 3
    assert session.run_raw(entry, p, ws) == abi.INVALID_ARGUMENT
    assert status(mode=abi.ATTENTION_PREFILL) == abi.INVALID_ARGUMENT  # the plan was made for decode
    p = d.params()
    p.kv_indices.length = 1
    assert session.run_raw(entry, p, ws) == abi.INVALID_ARGUMENT
    p = d.params()
    p.q.dtype = abi.DTYPE_F16
    assert session.run_raw(entry, p, ws) == abi.INVALID_ARGUMENT
    assert status(kv_layout=abi.LAYOUT_ROW_MAJOR) == abi.INVALID_ARGUMENT
    p = d.params()
    p.struct_size = 64
    assert session.run_raw(entry, p, ws) == abi.ABI_MISMATCH
    # plan without host tables; plan into a too-small workspace.
    p = d.params()
    p.kv_indptr_host = None
    assert entry.plan(session.ctx, C.addressof(p), C.addressof(ws), C.c_void_p(session.stream_handle)) == \
        abi.INVALID_ARGUMENT
    small = abi.new(abi.Workspace)
    small.device, small.device_bytes = ws.device, 64
    small.pinned_host, small.pinned_host_bytes = ws.pinned_host, 64
    small.plan, small.plan_bytes = ws.plan, ws.plan_bytes
    assert entry.plan(session.ctx, C.addressof(good), C.addressof(small), C.c_void_p(session.stream_handle)) == \
        abi.WORKSPACE_TOO_SMALL
    torch().cuda.synchronize()


# ---- Sliding window (CpuOps.cs:180-197, 245-252): query position pos sees keys j >= pos - window_left ---------------


def _release_before_window(b: cases.PagedBatch, window, causal=True):
    """Marks every page that no query of its sequence can see as released (-1), as the block manager does for blocks
    that left a sliding window (R-028): the kernels must neither read them nor fault on them."""
    idx = b.kv_indices.copy()
    for s in range(b.batch):
        n = int(b.q_indptr[s + 1] - b.q_indptr[s])
        first = max(0, int(b.kv_lens[s]) - n - window)  # the first query's first visible key
        for pi in range(int(b.kv_indptr[s]), int(b.kv_indptr[s + 1])):
            page = pi - int(b.kv_indptr[s])
            if (page + 1) * b.page_size <= first:
                idx[pi] = -1
    b.kv_indices = idx
    return b


WINDOW_DECODE_CASES = [
    ("decode w1", [5, 37, 130, 16], 16, False, 1),
    ("decode w40 ps16", [900, 17, 1, 2048, 333, 64, 1024, 777], 16, False, 40),
    ("decode w100 HND ps64", [900, 17, 1, 2048, 333, 64, 1024, 777], 64, True, 100),
    ("decode w4096 longer than most", [900, 6000, 5000, 40], 16, False, 4096),
    ("decode w33 ps7 general pages", [5, 37, 130, 1000], 7, False, 33),
]


@pytest.mark.parametrize("name,kv_lens,ps,hnd,window", WINDOW_DECODE_CASES, ids=[c[0] for c in WINDOW_DECODE_CASES])
def test_decode_sliding_window(session, name, kv_lens, ps, hnd, window):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = _release_before_window(cases.make_paged_batch(rng, kv_lens, [1] * len(kv_lens), page_size=ps, hnd=hnd),
                               window)
    got = run_case(session, b, window_left=window)
    check_against_oracle(got, b, window_left=window)


def test_decode_sliding_window_f32(session):
    """The f32 decode path (config 1's types) with a window and released pages."""
    rng = np.random.default_rng(41)
    b = _release_before_window(cases.make_paged_batch(rng, [17, 300, 120, 64], [1] * 4, bf16=False, d=64), 50)
    got = run_case(session, b, window_left=50)
    ref = cases.values(cases.oracle_attention(b, window_left=50), False)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


WINDOW_PREFILL_CASES = [
    ("prefill w128 fresh-700", [(700, 700)], 16, False, True, 128),
    ("prefill w1000 chunk-512-of-4000 split", [(512, 4000), (3, 3)], 16, False, True, 1000),
    ("prefill w64 multi-seq HND ps32", [(17, 17), (64, 300), (200, 200)], 32, True, True, 64),
    ("prefill w50 ps8 general", [(100, 300)], 8, False, True, 50),
    ("prefill w200 non-causal", [(32, 400)], 16, False, False, 200),
    ("prefill w300 mixed step", [(1, 900), (1, 17), (200, 1200), (1, 3000), (64, 64)], 16, False, True, 300),
    ("prefill w5000 wider than every context", [(128, 1000), (40, 40)], 16, False, True, 5000),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window", WINDOW_PREFILL_CASES,
                         ids=[c[0] for c in WINDOW_PREFILL_CASES])
def test_prefill_sliding_window(session, name, seqs, ps, hnd, causal, window):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd)
    if causal:
        b = _release_before_window(b, window)
    got = run_case(session, b, causal=causal, window_left=window)
    check_against_oracle(got, b, causal=causal, window_left=window)


def test_sliding_window_plan_must_match_run(session):
    """A plan made for one window is refused by a run with another (the pieces start at the window)."""
    rng = np.random.default_rng(77)
    b = cases.make_paged_batch(rng, [300, 40], [1, 1])
    d = Dev(b, window_left=64)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    session.launch(entry, d.params(), key="window")
    ws = session._ws[(entry.variant_id, "window")][3]
    d.window_left = -1
    assert session.run_raw(entry, d.params(), ws) == abi.INVALID_ARGUMENT


# ---- Prefill at head_dim 128 (the tile kernel templated on the head dim; decode already serves 64/128/256) ---------

HD128_PREFILL_CASES = [
    ("hd128 fresh-300", [(300, 300)], 16, False, True, -1),
    ("hd128 chunk-128-of-1000 HND ps32", [(128, 1000)], 32, True, True, -1),
    ("hd128 chunk-512-of-4000 split", [(512, 4000), (3, 3)], 16, False, True, -1),
    ("hd128 mixed step", [(1, 900), (1, 17), (200, 1200), (1, 3000), (64, 64)], 64, False, True, -1),
    ("hd128 non-causal-32-of-200", [(32, 200)], 16, False, False, -1),
    ("hd128 window 100", [(700, 700), (40, 900)], 16, False, True, 100),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window", HD128_PREFILL_CASES, ids=[c[0] for c in HD128_PREFILL_CASES])
def test_prefill_head_dim_128(session, name, seqs, ps, hnd, causal, window):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=128)
    got = run_case(session, b, causal=causal, window_left=window)
    check_against_oracle(got, b, causal=causal, window_left=window)


HD64_PREFILL_CASES = [
    ("hd64 fresh-300", [(300, 300)], 16, False, True, -1, 4),
    ("hd64 chunk-128-of-1000 HND ps32", [(128, 1000)], 32, True, True, -1, 4),
    ("hd64 chunk-512-of-4000 split", [(512, 4000), (3, 3)], 16, False, True, -1, 4),
    ("hd64 mixed step group 8", [(1, 900), (1, 17), (200, 1200), (1, 3000), (64, 64)], 64, False, True, -1, 8),
    ("hd64 non-causal-32-of-200", [(32, 200)], 16, False, False, -1, 4),
    ("hd64 window 100", [(700, 700), (40, 900)], 16, False, True, 100, 4),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window,group", HD64_PREFILL_CASES,
                         ids=[c[0] for c in HD64_PREFILL_CASES])
def test_prefill_head_dim_64(session, name, seqs, ps, hnd, causal, window, group):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=64,
                               hq=2 * group, hkv=2)
    got = run_case(session, b, causal=causal, window_left=window)
    check_against_oracle(got, b, causal=causal, window_left=window)


def test_prefill_head_dim_128_needs_a_dma_page_size(session):
    """Head dim 128 prefill is built on the DMA-fed tile kernel only: page sizes that are powers of two and multiples
    of 16. Page size 8 is refused as UNSUPPORTED before any launch."""
    rng = np.random.default_rng(5)
    b = cases.make_paged_batch(rng, [100], [50], page_size=8, d=128)
    d = Dev(b)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    sizes = abi.new(abi.WorkspaceSizes)
    params = d.params()  # held here: the call reads it through a raw address
    assert entry.workspace(session.ctx, C.addressof(params), C.addressof(sizes)) == abi.UNSUPPORTED


# ---- Groups of 8, 16 and 32 query heads per KV head: 2, 4 or 8 groups of 4 reading the same KV rows -----------------

GROUP_CASES = [
    ("decode group 8", "decode", [900, 17, 1, 2048, 333, 64], 16, False, 16, 2, 256),
    ("decode group 16 HND ps64", "decode", [900, 17, 2048, 64], 64, True, 32, 2, 128),
    ("decode group 8 ps7 general pages", "decode", [5, 37, 130, 1000], 7, False, 8, 1, 128),
    ("prefill group 8", "prefill", [(300, 300), (64, 700)], 16, False, 16, 2, 256),
    ("prefill group 32 hd128", "prefill", [(200, 1200)], 32, False, 32, 1, 128),
    ("prefill group 8 mixed step", "prefill", [(1, 900), (130, 700), (1, 40)], 16, False, 16, 2, 256),
]


@pytest.mark.parametrize("name,mode,lens,ps,hnd,hq,hkv,d", GROUP_CASES, ids=[c[0] for c in GROUP_CASES])
def test_query_head_groups(session, name, mode, lens, ps, hnd, hq, hkv, d):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    if mode == "decode":
        b = cases.make_paged_batch(rng, lens, [1] * len(lens), page_size=ps, hnd=hnd, hq=hq, hkv=hkv, d=d)
    else:
        b = cases.make_paged_batch(rng, [s[1] for s in lens], [s[0] for s in lens], page_size=ps, hnd=hnd, hq=hq,
                                   hkv=hkv, d=d)
    got = run_case(session, b)
    check_against_oracle(got, b)


# ---- plan() without kv_last_page_len_host ---------------------------------------------------------------------------
# The reference's plan() needs only the q and kv indptr host tables (kernels/src/paged_attention.cu:107); the kernels
# must then take every sequence's key count from the device's kv_last_page_len. With partial last pages the plan's
# assumption (full pages) is wrong by up to page_size - 1 keys.

NOLAST_CASES = [
    ("non-causal hd256", [(32, 203), (70, 1001)], 16, False, False, -1, 256),
    ("non-causal hd256 split", [(512, 4001), (3, 9)], 16, False, False, -1, 256),
    ("causal hd256 split", [(512, 4001), (100, 233)], 16, False, True, -1, 256),
    ("windowed hd256", [(300, 1201), (64, 77)], 16, False, True, 100, 256),
    ("windowed hd256 split", [(512, 4001)], 16, False, True, 1500, 256),
    ("windowed non-causal hd256 ps32", [(40, 505)], 32, False, False, 200, 256),
    ("non-causal hd128", [(32, 203), (70, 1001)], 16, False, False, -1, 128),
    ("windowed hd128 HND split", [(512, 4001), (64, 77)], 16, True, True, 1000, 128),
    ("mixed step with decode rows", [(1, 901), (130, 705), (1, 4003)], 16, False, True, -1, 256),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window,d", NOLAST_CASES, ids=[c[0] for c in NOLAST_CASES])
def test_prefill_plan_without_last_page_len_host(session, name, seqs, ps, hnd, causal, window, d):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=d)
    assert any(int(x) < ps for x in b.kv_last_page_len), "the case needs a partial last page"
    dv = Dev(b, causal, window_left=window)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    session.launch(entry, dv.params(kv_last_page_len_host=None), key=("nolast", name))
    check_against_oracle(dv.result(), b, causal=causal, window_left=window)


# ---- Logit soft capping (CpuOps.cs:276; the reference GPU library refuses it, kernels/src/paged_attention.cu:92-94) --

SOFTCAP_CASES = [
    ("decode bf16 hd256", [(1, 700), (1, 33), (1, 1500)], 16, False, True, 256, True, 5.0),
    ("decode bf16 hd64 HND ps64", [(1, 300), (1, 901)], 64, True, True, 64, True, 3.0),
    ("decode bf16 hd128 split", [(1, 6000)], 16, False, True, 128, True, 8.0),
    ("decode f32 hd64", [(1, 200), (1, 77)], 16, False, True, 64, False, 4.0),
    ("prefill hd256 split", [(512, 4000), (3, 3)], 16, False, True, 256, True, 5.0),
    ("prefill hd128 non-causal", [(40, 300)], 16, False, False, 128, True, 2.0),
    ("prefill ps8 general", [(100, 300)], 8, False, True, 256, True, 5.0),
    ("mixed step", [(1, 900), (200, 1200), (1, 3000), (64, 64)], 16, False, True, 256, True, 30.0),
    ("prefill f32 hd128", [(30, 200), (1, 50)], 16, False, True, 128, False, 4.0),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,d,bf16,cap", SOFTCAP_CASES, ids=[c[0] for c in SOFTCAP_CASES])
def test_logit_soft_cap(session, name, seqs, ps, hnd, causal, d, bf16, cap):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    # std 2 puts the scaled scores at a few units, where a cap of 2-8 bends them; a negative cap caps alike.
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=d,
                               bf16=bf16, std=2.0)
    dv = Dev(b, causal, soft_cap=-cap if "HND" in name else cap)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    session.launch(entry, dv.params(), key=("softcap", name))
    got = dv.result()
    ref = cases.values(cases.oracle_attention(b, causal, soft_cap=cap), b.bf16)
    if bf16:
        # V is drawn at std 2 as well, so outputs and their bf16 steps are twice the std-1 cases': the absolute
        # tolerance scales with them.
        cases.assert_close(got, ref, max_abs=2 * cases.MAX_ABS, what=f"soft cap {name}")
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # The cap changes the result (the case exercises it).
    uncapped = cases.values(cases.oracle_attention(b, causal), b.bf16)
    assert np.abs(uncapped - ref).max() > 1e-2


# ---- f32 prefill (CpuOps.cs:198-298 computes in any dtype; the reference GPU library refuses it) ----------------------
#
# No f32 MFMA tile kernel: every query token becomes a row of the f32 decode kernel (its position, causal end and
# window start), rows longer than a range are split and merged like decode rows. Checked against CpuOps at f32's own
# accuracy (fp32 accumulation against the oracle's double).

F32_PREFILL_CASES = [
    ("causal hd256 mixed lengths", [(37, 300), (1, 90), (64, 64)], 16, False, True, -1, 256),
    ("non-causal hd128 HND", [(20, 180), (5, 33)], 16, True, False, -1, 128),
    ("window hd64 page size 7", [(50, 400), (1, 77)], 7, False, True, 100, 64),
    ("non-causal window hd256 ps32", [(30, 500)], 32, False, False, 64, 256),
    ("long rows split and merged", [(6, 9000), (3, 40)], 16, False, True, -1, 256),
]


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window,d", F32_PREFILL_CASES, ids=[c[0] for c in F32_PREFILL_CASES])
def test_prefill_f32_matches_cpuops(session, name, seqs, ps, hnd, causal, window, d):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=d,
                               bf16=False)
    got = run_case(session, b, causal, window_left=window)
    ref = cases.values(cases.oracle_attention(b, causal, window_left=window), False)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def test_decode_large_batch(session):
    """8,192 decode rows of 1 to 64 keys (far more sequences than ranges) against a float32 torch reference."""
    rng = np.random.default_rng(77)
    kv = rng.integers(1, 65, size=8192)
    b = cases.make_paged_batch(rng, kv, np.ones(8192, np.int64), std=0.5)
    got = run_case(session, b, check_nohost=False, check_determinism=False)
    cases.assert_close(got, torch_reference(b), what="8192-row decode vs fp32 torch")


def test_prefill_long_sequence_sampled_rows(session):
    """One causal prefill of 32,768 tokens (hundreds of pieces and merges at head dim 256): sampled query rows -- the
    first, tile and piece edges, the last -- against a float64 numpy evaluation of those rows alone."""
    rng = np.random.default_rng(78)
    L = 32768
    b = cases.make_paged_batch(rng, [L], [L], std=0.5)
    got = run_case(session, b, check_nohost=False, check_determinism=False)
    vals = lambda a: cases.values(a, True).astype(np.float64)  # noqa: E731
    q, kc, vc = vals(b.q), vals(b.k_cache), vals(b.v_cache)
    pos = np.arange(L)
    page, slot = b.kv_indices[pos // b.page_size], pos % b.page_size
    k = kc[page, slot]  # [L, hkv, d]
    v = vc[page, slot]
    scale = 1.0 / np.sqrt(b.d)
    group = b.hq // b.hkv
    for t in (0, 63, 64, 1000, 4095, 4096, 20000, L - 1):
        for h in range(b.hq):
            s = (k[: t + 1, h // group] @ q[t, h]) * scale
            p = np.exp(s - s.max())
            ref = (p @ v[: t + 1, h // group]) / p.sum()
            cases.assert_close(got[t, h][None], ref[None], what=f"32k prefill row {t} head {h}")


def _random_case(rng):
    """One random paged call: batch 1-6, decode rows (one token) mixed with prefill chunks on random prefixes, head
    dims 64/128/256, page sizes 7/16/32/64, NHD or HND, causal or not, with or without a window and a soft cap."""
    d = int(rng.choice([64, 128, 256]))
    ps = int(rng.choice([16, 32, 64] + ([7] if d == 256 else [])))  # head dims 64 and 128 prefill need the DMA pages
    batch = int(rng.integers(1, 7))
    decode = rng.random() < 0.3
    q_lens = [1 if decode or rng.random() < 0.3 else int(rng.integers(2, 300)) for _ in range(batch)]
    kv_lens = [q + int(rng.integers(0, 900)) for q in q_lens]
    causal = bool(rng.random() < 0.7)
    window = -1 if rng.random() < 0.6 else int(rng.integers(30, 500))
    cap = 0.0 if rng.random() < 0.7 else float(rng.choice([5.0, 20.0]))
    return dict(d=d, ps=ps, q_lens=q_lens, kv_lens=kv_lens, hnd=bool(rng.random() < 0.5), causal=causal,
                window=window, cap=cap)


@pytest.mark.parametrize("seed", range(64))
def test_random_attention_calls_match_cpuops(session, seed):
    """Random combinations of the call's features (decode and prefill rows in one batch, head dims, page sizes, layouts,
    causal or not, window, soft cap) against CpuOps, with the same bf16 tolerance as the fixed cases."""
    rng = np.random.default_rng(1000 + seed)
    c = _random_case(rng)
    b = cases.make_paged_batch(rng, c["kv_lens"], c["q_lens"], page_size=c["ps"], hnd=c["hnd"], d=c["d"], std=0.5)
    mode = abi.ATTENTION_DECODE if all(q == 1 for q in c["q_lens"]) else abi.ATTENTION_PREFILL
    dev = Dev(b, c["causal"], window_left=c["window"], soft_cap=c["cap"])
    print(f"seed {seed}: {c}", flush=True)
    session.launch(session.lib.entry(roost_amd.ATTENTION_VARIANT), dev.params(mode=mode), key=("random", seed))
    got = dev.result()
    ref = cases.values(cases.oracle_attention(b, c["causal"], window_left=c["window"], soft_cap=c["cap"]), True)
    cases.assert_close(got, ref, what=f"random attention {seed}")
    cases.assert_attention_class(got, ref, float(np.abs(cases.values(b.v_cache, True)).max()),
                                 what=f"random attention {seed}")
