"""Benchmark of the gfx950 Roost attention + Gated DeltaNet kernel library on one MI355X.

Headline (BASELINE.json metric, `value`): paged bf16 decode attention at BASELINE config 2 -- Qwen3.5-0.8B shape,
batch 64, contexts U(512, 8192), 8 query / 2 KV heads, head_dim 256, page 16, pool 1.25x tokens -- as achieved HBM
GB/s over the algorithmic bytes (K and V of every context token, q read and o write, the page tables). A step is one
run() of the PagedAttention entry point over the batch, inputs resident in HBM, plan() done beforehand (it is a host
step, timed separately). The same JSON line carries config 3 causal chunked prefill (TFLOP/s vs bf16 dense MFMA peak),
config 4 GDN chunked prefill and recurrent decode, the roofline of the dominant decode kernel, and the CpuOps oracle
timed on the host as the CPU baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
METRIC = "decode attn HBM GB/s (% peak) + prefill TFLOPS (% MFMA peak) vs CpuOps, 1 GPU"
FLUSH = None  # the cache-flush buffer (set in main)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class Paged:
    """A seeded paged batch built directly on the device (host copies only of the small tables)."""

    def __init__(self, torch, rng, kv_lens, q_lens, std=0.5, hq=8, hkv=2, d=256, ps=16, pool_factor=1.25):
        self.kv_lens = np.asarray(kv_lens, np.int64)
        self.q_lens = np.asarray(q_lens, np.int64)
        pages = (self.kv_lens + ps - 1) // ps
        total = int(pages.sum())
        pool = int(np.ceil(total * pool_factor))
        self.kv_indices_h = rng.permutation(pool)[:total].astype(np.int32)
        self.q_indptr_h = np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)
        self.kv_indptr_h = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
        self.last_h = (self.kv_lens - (pages - 1) * ps).astype(np.int32)
        self.tokens = int(self.q_indptr_h[-1])
        self.batch = len(kv_lens)
        self.hq, self.hkv, self.d, self.ps, self.pages, self.pool = hq, hkv, d, ps, total, pool
        g = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 31)))
        self.q = (torch.randn((self.tokens, hq, d), generator=g, device="cuda") * std).to(torch.bfloat16)
        self.k = (torch.randn((pool, ps, hkv, d), generator=g, device="cuda") * std).to(torch.bfloat16)
        self.v = (torch.randn((pool, ps, hkv, d), generator=g, device="cuda") * std).to(torch.bfloat16)
        dev = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
        self.q_indptr, self.kv_indptr = dev(self.q_indptr_h), dev(self.kv_indptr_h)
        self.kv_indices, self.last = dev(self.kv_indices_h), dev(self.last_h)
        self.out = torch.empty_like(self.q)

    def params(self, roost_amd, causal=True):
        return roost_amd.paged_attention_params(
            self.q, self.out, self.k, self.v, self.q_indptr, self.kv_indptr, self.kv_indices, self.last,
            q_indptr_host=self.q_indptr_h, kv_indptr_host=self.kv_indptr_h, kv_last_page_len_host=self.last_h,
            batch=self.batch, q_heads=self.hq, kv_heads=self.hkv, head_dim=self.d, page_size=self.ps, causal=causal)

    def decode_bytes(self):
        e = 2
        kv = int(self.kv_lens.sum()) * self.hkv * self.d * 2 * e
        qo = self.batch * self.hq * self.d * 2 * e
        tables = 4 * (self.pages + 2 * self.batch + 1)
        return kv + qo + tables

    def prefill_flops(self):
        n, p = self.q_lens, self.kv_lens - self.q_lens
        return float(4 * self.hq * self.d * np.sum(n * p + n * (n + 1) / 2))


def time_runs(torch, session, entry, params, ws, steps, warmup):
    """Average run() duration in ms over `steps` launches, measured with events on the session's stream, after
    settling the GPU on the same call."""
    settle(session, lambda: session.run(entry, params, ws))
    for _ in range(warmup):
        session.run(entry, params, ws)
    session.stream.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(session.stream)
    for _ in range(steps):
        session.run(entry, params, ws)
    end.record(session.stream)
    end.synchronize()
    return start.elapsed_time(end) / steps


class Flush:
    """A 512 MiB device buffer read between timed launches: it evicts the 256 MB MALL and the L2s with clean lines,
    so a cold launch reads its inputs from HBM (a written buffer would instead leave dirty lines whose write-back
    lands inside the timed launch)."""

    def __init__(self, torch):
        self.buf = torch.ones(128 << 20, dtype=torch.int32, device="cuda")

    def __call__(self, stream):
        import torch

        with torch.cuda.stream(stream):
            self.sink = self.buf.sum()


def time_cold(torch, session, flush, fn, reps):
    """Median duration in ms of `fn` (launches on the session's stream), each launch timed alone with events after a
    cache flush."""
    times = []
    for _ in range(reps):
        flush(session.stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(session.stream)
        fn()
        e1.record(session.stream)
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return float(np.median(times))


SETTLE_S = 0.3  # --settle


def settle(session, fn, seconds=None):
    """Runs `fn` back to back for `seconds` (default --settle) so that clocks and caches reach their steady state before
    a timing."""
    seconds = SETTLE_S if seconds is None else seconds
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        session.stream.synchronize()


def time_each(torch, session, fn, reps, warmup=2):
    """Median duration in ms of `fn` launched back to back (warm caches), each launch between its own events, after
    settling the GPU on it."""
    settle(session, fn)
    for _ in range(warmup):
        fn()
    session.stream.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in evs:
        e0.record(session.stream)
        fn()
        e1.record(session.stream)
    evs[-1][1].synchronize()
    return float(np.median([e0.elapsed_time(e1) for e0, e1 in evs]))


def planned(session, entry, params, key, reps=20):
    """Workspace + plan, returning the workspace and the host cost of one step's planning in ms: the workspace query
    and plan() (host tables, pinned staging, async copy) as the worker calls them every step, averaged over `reps`
    once the buffers exist (the first launch also allocates them and is not counted)."""
    import ctypes as C

    session.launch(entry, params, key=key)  # allocates, plans and runs once
    session.stream.synchronize()
    slot = session._ws.get((entry.variant_id, key))
    if slot is None:
        return None, 0.0
    ws = slot[3]
    if not entry.needs_plan:
        return ws, 0.0
    t0 = time.perf_counter()
    for _ in range(reps):
        session.workspace_sizes(entry, params)
        status = entry.plan(session.ctx, C.addressof(params), C.addressof(ws), C.c_void_p(session.stream_handle))
        assert status == 0, status
        session.stream.synchronize()  # the pinned staging buffer is reused by the next plan
    plan_ms = (time.perf_counter() - t0) * 1e3 / reps
    return ws, plan_ms


def bench_decode(torch, roost_amd, session, steps, warmup):
    rng = np.random.default_rng(2)
    kv = rng.integers(512, 8193, size=64)
    b = Paged(torch, rng, kv, np.ones(64, np.int64))
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    p = b.params(roost_amd)
    ws, plan_ms = planned(session, entry, p, "bench-decode")
    ms = time_runs(torch, session, entry, p, ws, steps, warmup)
    if FLUSH is not None:
        b.cold_ms = time_cold(torch, session, FLUSH, lambda: session.run(entry, p, ws), 10)
    return b, ms, plan_ms


def bench_prefill(torch, roost_amd, session, steps, warmup, d=256):
    """Config 3's draw (seed 3); d=128 runs the same batch at head dim 128 (the second tile-kernel instantiation)."""
    rng = np.random.default_rng(3)
    n = rng.integers(256, 2049, size=8)
    pre = rng.integers(0, 6145, size=8)
    b = Paged(torch, rng, n + pre, n, d=d)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    p = b.params(roost_amd)
    ws, plan_ms = planned(session, entry, p, "bench-prefill")
    reps = max(steps // 2, 20)
    ms = time_each(torch, session, lambda: session.run(entry, p, ws), reps)
    # The config's step also writes the chunks' new K/V rows into their (freshly allocated, random) pages first:
    # CacheWrite at the plan-region slots, then the attention call.
    slots_h = []
    for i in range(b.batch):
        pages = b.kv_indices_h[b.kv_indptr_h[i]:b.kv_indptr_h[i + 1]].astype(np.int64)
        pos = np.arange(b.kv_lens[i] - b.q_lens[i], b.kv_lens[i])
        slots_h.append(pages[pos // b.ps] * b.ps + pos % b.ps)
    g = torch.Generator(device="cuda").manual_seed(33)
    new_k = (torch.randn((b.tokens, b.hkv, b.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    new_v = (torch.randn((b.tokens, b.hkv, b.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    cw = roost_amd.cache_write_params(new_k, new_v, b.k, b.v, torch.from_numpy(np.concatenate(slots_h)).cuda(),
                                      kv_heads=b.hkv, head_dim=b.d, page_size=b.ps)
    e_cw = session.lib.entry(roost_amd.CACHE_WRITE_VARIANT)

    def step():
        session.run(e_cw, cw, None)
        session.run(entry, p, ws)

    b.append_ms = time_each(torch, session, step, reps)
    return b, ms, plan_ms


def bench_gdn(torch, roost_amd, session, steps, warmup):
    H, D = 16, 128
    g = torch.Generator(device="cuda").manual_seed(4)

    def inputs(batch, lens):
        tokens = int(sum(lens))
        fused = torch.randn((tokens, 3 * H * D), generator=g, device="cuda").to(torch.bfloat16)
        gg = -torch.nn.functional.softplus(torch.randn((tokens, H), generator=g, device="cuda"))
        beta = torch.sigmoid(torch.randn((tokens, H), generator=g, device="cuda")).to(torch.bfloat16)
        pool = torch.randn((batch, H, D, D), generator=g, device="cuda") * 0.01
        slots = torch.arange(batch, dtype=torch.int32, device="cuda")
        cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        out = torch.empty((tokens, H, D), dtype=torch.bfloat16, device="cuda")
        reach = (tokens - 1) * 3 * H * D + H * D
        p = roost_amd.gated_delta_rule_params(
            fused, fused, fused, gg, beta, out, pool, slots, torch.from_numpy(cu_h).cuda(), batch=batch,
            tokens=tokens, q_stride=3 * H * D, k_stride=3 * H * D, v_stride=3 * H * D, q_len=reach, k_len=reach,
            v_len=reach, q_offset=0, k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h)
        return p, (fused, gg, beta, pool, slots, out)

    res = {}
    # Config 4: chunked prefill, 4 x 4096 tokens.
    p, keep = inputs(4, [4096] * 4)
    entry = session.lib.entry(roost_amd.CHUNK_VARIANT)
    ws, _ = planned(session, entry, p, "bench-gdn-chunk")
    run = lambda: session.run(entry, p, ws)  # noqa: E731
    ms = time_each(torch, session, run, max(steps // 2, 10))
    cold = time_cold(torch, session, FLUSH, run, 10) if FLUSH is not None else None
    T, B, C = 4 * 4096, 4, 64
    bytes_ = (3 * T * H * D + T * H * D) * 2 + T * H * 6 + 2 * B * H * D * D * 4
    # Algorithmic flops of the WY form per chunk of C = 64 tokens and head: 2 C^2 (3 dk + 2 dv) + 6 C dk dv
    # (11.53 MFLOP; the bf16 hi / lo operand splits are not counted).
    flops = (T // C) * H * (2 * C * C * (3 * D + 2 * D) + 6 * C * D * D)
    res["gdn_chunk"] = {"config": "4 x 4096 tokens, 16 heads x 128, chunk 64", "ms": ms, "cold_ms": cold,
                        "hbm_gbs": bytes_ / ms / 1e6, "hbm_frac": bytes_ / ms / 1e6 / HBM_PEAK_GBS,
                        "tflops": flops / ms / 1e9, "mfma_frac": flops / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                        "flops": flops, "algorithmic_bytes": bytes_}
    del keep
    # Config 4 follow-on: one recurrent decode step on 128 states.
    p, keep = inputs(128, [1] * 128)
    entry = session.lib.entry(roost_amd.RECURRENT_VARIANT)
    ws, _ = planned(session, entry, p, "bench-gdn-recurrent")
    ms = time_runs(torch, session, entry, p, ws, steps, warmup)
    cold = time_cold(torch, session, FLUSH, lambda: session.run(entry, p, ws), 10) if FLUSH is not None else None
    B = 128
    bytes_ = 2 * B * H * D * D * 4 + B * (3 * H * D + H * D) * 2 + B * H * 6
    res["gdn_recurrent"] = {"config": "128 states x 1 token, 16 heads x 128", "ms": ms, "cold_ms": cold,
                            "hbm_gbs": bytes_ / ms / 1e6, "hbm_frac": bytes_ / ms / 1e6 / HBM_PEAK_GBS,
                            "cold_hbm_frac": bytes_ / cold / 1e6 / HBM_PEAK_GBS if cold else None}
    del keep
    res["gdn_decode_layer"] = bench_decode_layer(torch, roost_amd, session, steps, g)
    res["gdn_chunk_layer"] = bench_chunk_layer(torch, roost_amd, session, steps, g)
    res["gdn_step_layer"] = bench_step_layer(torch, roost_amd, session, steps, g)
    return res


def bench_step_layer(torch, roost_amd, session, steps, g):
    """Config 5's GDN layer as a whole Qwen3.5 layer (CausalConv1d of width 4 over the 6,144-channel projection,
    GatedDeltaRuleGates, the recurrent GatedDeltaRule routing the two 512-token chunks to the chunk kernels,
    GatedRmsNorm; 48 one-token sequences and 2 x 512 tokens): the four ops one after another against
    roost_amd_gdn_layer_run."""
    H, D, W = 16, 128, 4
    lens = np.array([1] * 48 + [512, 512])
    B, T, ch = len(lens), int(lens.sum()), 3 * H * D
    bf = lambda t: t.to(torch.bfloat16)  # noqa: E731
    x = bf(torch.randn((T, ch), generator=g, device="cuda"))
    w = bf(torch.randn((ch, W), generator=g, device="cuda") * 0.5)
    bias = bf(torch.randn((ch,), generator=g, device="cuda") * 0.3)
    conv_state = bf(torch.randn((B, ch, W - 1), generator=g, device="cuda"))
    slots = torch.arange(B, dtype=torch.int32, device="cuda")
    cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cu = torch.from_numpy(cu_h).cuda()
    y = torch.empty((T, ch), dtype=torch.bfloat16, device="cuda")
    proj = bf(torch.randn((T, 2 * H), generator=g, device="cuda") * 3)
    a_log = torch.randn((H,), generator=g, device="cuda") * 0.5
    dt_bias = torch.randn((H,), generator=g, device="cuda")
    gg = torch.empty((T, H), dtype=torch.float32, device="cuda")
    beta = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    pool = torch.randn((B, H, D, D), generator=g, device="cuda") * 0.01
    o = torch.empty((T, H, D), dtype=torch.bfloat16, device="cuda")
    z = bf(torch.randn((T * H, D), generator=g, device="cuda"))
    nw = 1 + torch.randn((D,), generator=g, device="cuda") * 0.2
    out = torch.empty((T * H, D), dtype=torch.bfloat16, device="cuda")
    conv = roost_amd.causal_conv1d_params(x, w, bias, y, conv_state, slots, cu, batch=B, tokens=T, channels=ch, width=W)
    gkw = dict(tokens=T, v_heads=H, a_stride=2 * H, b_stride=2 * H, a_len=(T - 1) * 2 * H + H,
               b_len=(T - 1) * 2 * H + H, a_offset=H, b_offset=0)
    gates = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, gg, beta, **gkw)
    gates_in = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, None, None, **gkw)
    reach = (T - 1) * ch + H * D

    def gdn_params(gv, bv):
        return roost_amd.gated_delta_rule_params(
            y, y, y, gv, bv, o, pool, slots, cu, batch=B, tokens=T, q_stride=ch, k_stride=ch, v_stride=ch, q_len=reach,
            k_len=reach, v_len=reach, q_offset=0, k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h)

    gdn, gdn_in = gdn_params(gg, beta), gdn_params(None, None)
    norm = roost_amd.gated_rms_norm_params(o, z, nw, out, rows=T * H, dim=D, eps=1e-6)
    e_conv = session.lib.entry(roost_amd.CAUSAL_CONV1D_VARIANT)
    e_gates = session.lib.entry(roost_amd.GATES_VARIANT)
    e_gdn = session.lib.entry(roost_amd.RECURRENT_VARIANT)
    e_norm = session.lib.entry(roost_amd.GATED_RMS_NORM_VARIANT)
    ws_gdn, _ = planned(session, e_gdn, gdn, "bench-step-layer-gdn")

    def four():
        session.run(e_conv, conv, None)
        session.run(e_gates, gates, None)
        session.run(e_gdn, gdn, ws_gdn)
        session.run(e_norm, norm, None)

    def fused():
        roost_amd.gdn_layer(session, conv, gates_in, gdn_in, norm, key="bench-step")

    return {"config": "config 5's GDN layer: 48 x 1 + 2 x 512 tokens, Qwen3.5 layer (conv width 4, gates, recurrent "
                      "variant, gated norm)",
            "four_ops_ms": time_each(torch, session, four, steps), "fused_ms": time_each(torch, session, fused, steps)}


def bench_chunk_layer(torch, roost_amd, session, steps, g):
    """Config 4's prefill as a whole Qwen3.5 GDN layer (CausalConv1d of width 4 over the 6,144-channel q|k|v projection,
    GatedDeltaRuleGates, the chunked GatedDeltaRule, GatedRmsNorm; 4 x 4096 tokens): the four ops one after another
    (the chunk variant for the GDN op) against roost_amd_gdn_chunk_layer_run."""
    H, D, B, W, n = 16, 128, 4, 4, 4096
    T, ch = B * n, 3 * H * D
    bf = lambda t: t.to(torch.bfloat16)  # noqa: E731
    x = bf(torch.randn((T, ch), generator=g, device="cuda"))
    w = bf(torch.randn((ch, W), generator=g, device="cuda") * 0.5)
    bias = bf(torch.randn((ch,), generator=g, device="cuda") * 0.3)
    conv_state = bf(torch.randn((B, ch, W - 1), generator=g, device="cuda"))
    slots = torch.arange(B, dtype=torch.int32, device="cuda")
    cu_h = (np.arange(B + 1) * n).astype(np.int32)
    cu = torch.from_numpy(cu_h).cuda()
    y = torch.empty((T, ch), dtype=torch.bfloat16, device="cuda")
    proj = bf(torch.randn((T, 2 * H), generator=g, device="cuda") * 3)
    a_log = torch.randn((H,), generator=g, device="cuda") * 0.5
    dt_bias = torch.randn((H,), generator=g, device="cuda")
    gg = torch.empty((T, H), dtype=torch.float32, device="cuda")
    beta = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    pool = torch.randn((B, H, D, D), generator=g, device="cuda") * 0.01
    o = torch.empty((T, H, D), dtype=torch.bfloat16, device="cuda")
    z = bf(torch.randn((T * H, D), generator=g, device="cuda"))
    nw = 1 + torch.randn((D,), generator=g, device="cuda") * 0.2
    out = torch.empty((T * H, D), dtype=torch.bfloat16, device="cuda")
    conv = roost_amd.causal_conv1d_params(x, w, bias, y, conv_state, slots, cu, batch=B, tokens=T, channels=ch, width=W)
    gkw = dict(tokens=T, v_heads=H, a_stride=2 * H, b_stride=2 * H, a_len=(T - 1) * 2 * H + H,
               b_len=(T - 1) * 2 * H + H, a_offset=H, b_offset=0)
    gates = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, gg, beta, **gkw)
    gates_in = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, None, None, **gkw)
    reach = (T - 1) * ch + H * D

    def gdn_params(gv, bv):
        return roost_amd.gated_delta_rule_params(
            y, y, y, gv, bv, o, pool, slots, cu, batch=B, tokens=T, q_stride=ch, k_stride=ch, v_stride=ch, q_len=reach,
            k_len=reach, v_len=reach, q_offset=0, k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h)

    gdn, gdn_in = gdn_params(gg, beta), gdn_params(None, None)
    norm = roost_amd.gated_rms_norm_params(o, z, nw, out, rows=T * H, dim=D, eps=1e-6)
    e_conv = session.lib.entry(roost_amd.CAUSAL_CONV1D_VARIANT)
    e_gates = session.lib.entry(roost_amd.GATES_VARIANT)
    e_gdn = session.lib.entry(roost_amd.CHUNK_VARIANT)
    e_norm = session.lib.entry(roost_amd.GATED_RMS_NORM_VARIANT)
    ws_gdn, _ = planned(session, e_gdn, gdn, "bench-chunk-layer-gdn")

    def four():
        session.run(e_conv, conv, None)
        session.run(e_gates, gates, None)
        session.run(e_gdn, gdn, ws_gdn)
        session.run(e_norm, norm, None)

    roost_amd.gdn_chunk_layer(session, conv, gates_in, gdn_in, norm, key="bench")  # workspace and plan

    def fused():
        roost_amd.gdn_chunk_layer(session, conv, gates_in, gdn_in, norm, key="bench", plan=False)

    reps = max(steps // 2, 10)
    four_ms = time_each(torch, session, four, reps)
    fused_ms = time_each(torch, session, fused, reps)
    return {"config": "4 x 4096 tokens, Qwen3.5 GDN layer (conv width 4, gates, chunked GDN, gated norm)",
            "four_ops_ms": four_ms, "fused_ms": fused_ms}


def bench_decode_layer(torch, roost_amd, session, steps, g):
    """The same decode step as a whole Qwen3.5 GDN layer (CausalConv1d of width 4 over the 6,144-channel q|k|v
    projection, GatedDeltaRuleGates, the recurrent GatedDeltaRule, GatedRmsNorm; 128 states x 1 token): the four ops one
    after another against roost_amd_gdn_decode_layer_run."""
    H, D, B, W = 16, 128, 128, 4
    ch = 3 * H * D
    bf = lambda t: t.to(torch.bfloat16)  # noqa: E731
    x = bf(torch.randn((B, ch), generator=g, device="cuda"))
    w = bf(torch.randn((ch, W), generator=g, device="cuda") * 0.5)
    bias = bf(torch.randn((ch,), generator=g, device="cuda") * 0.3)
    conv_state = bf(torch.randn((B, ch, W - 1), generator=g, device="cuda"))
    slots = torch.arange(B, dtype=torch.int32, device="cuda")
    cu_h = np.arange(B + 1, dtype=np.int32)
    cu = torch.from_numpy(cu_h).cuda()
    y = torch.empty((B, ch), dtype=torch.bfloat16, device="cuda")
    proj = bf(torch.randn((B, 2 * H), generator=g, device="cuda") * 3)
    a_log = torch.randn((H,), generator=g, device="cuda") * 0.5
    dt_bias = torch.randn((H,), generator=g, device="cuda")
    gg = torch.empty((B, H), dtype=torch.float32, device="cuda")
    beta = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    pool = torch.randn((B, H, D, D), generator=g, device="cuda") * 0.01
    o = torch.empty((B, H, D), dtype=torch.bfloat16, device="cuda")
    z = bf(torch.randn((B * H, D), generator=g, device="cuda"))
    nw = 1 + torch.randn((D,), generator=g, device="cuda") * 0.2
    out = torch.empty((B * H, D), dtype=torch.bfloat16, device="cuda")
    conv = roost_amd.causal_conv1d_params(x, w, bias, y, conv_state, slots, cu, batch=B, tokens=B, channels=ch, width=W)
    gkw = dict(tokens=B, v_heads=H, a_stride=2 * H, b_stride=2 * H, a_len=(B - 1) * 2 * H + H,
               b_len=(B - 1) * 2 * H + H, a_offset=H, b_offset=0)
    gates = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, gg, beta, **gkw)
    gates_in = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, None, None, **gkw)
    reach = (B - 1) * ch + H * D

    def gdn_params(gv, bv):
        return roost_amd.gated_delta_rule_params(
            y, y, y, gv, bv, o, pool, slots, cu, batch=B, tokens=B, q_stride=ch, k_stride=ch, v_stride=ch, q_len=reach,
            k_len=reach, v_len=reach, q_offset=0, k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h)

    gdn, gdn_in = gdn_params(gg, beta), gdn_params(None, None)
    norm = roost_amd.gated_rms_norm_params(o, z, nw, out, rows=B * H, dim=D, eps=1e-6)
    e_conv = session.lib.entry(roost_amd.CAUSAL_CONV1D_VARIANT)
    e_gates = session.lib.entry(roost_amd.GATES_VARIANT)
    e_gdn = session.lib.entry(roost_amd.RECURRENT_VARIANT)
    e_norm = session.lib.entry(roost_amd.GATED_RMS_NORM_VARIANT)
    ws_gdn, _ = planned(session, e_gdn, gdn, "bench-layer-gdn")

    def four():
        session.run(e_conv, conv, None)
        session.run(e_gates, gates, None)
        session.run(e_gdn, gdn, ws_gdn)
        session.run(e_norm, norm, None)

    def fused():
        roost_amd.gdn_decode_layer(session, conv, gates_in, gdn_in, norm)

    four_ms = time_each(torch, session, four, steps)
    fused_ms = time_each(torch, session, fused, steps)
    # Bytes of the fused call: the states read and written, the conv states read and written, x, z and the output.
    bytes_ = 2 * B * H * D * D * 4 + 2 * B * ch * (W - 1) * 2 + B * ch * 2 + 2 * B * H * D * 2 + B * 2 * H * 2
    return {"config": "128 states x 1 token, Qwen3.5 GDN layer (conv width 4, gates, recurrence, gated norm)",
            "four_ops_ms": four_ms, "fused_ms": fused_ms, "fused_hbm_frac": bytes_ / fused_ms / 1e6 / HBM_PEAK_GBS,
            "algorithmic_bytes": bytes_}


def bench_mixed(torch, roost_amd, session, steps, warmup):
    """one worker step of a 3:1 GDN:attention layer group. 48 decode sequences (contexts
    U(1024, 16384)) and 2 prefill chunks of 512 tokens on 4096-token prefixes share one paged KV pool and one state
    pool. The step is CacheWrite of the 1072 new tokens, one PagedAttention call (prefill mode, as the worker issues a
    mixed batch: tokens > batch) and three GatedDeltaRule calls on the recurrent variant (the one the worker names for
    every length), each layer with its own state slots. Returns the step latency and the per-op breakdown."""
    H, D = 16, 128
    rng = np.random.default_rng(5)
    dec = rng.integers(1024, 16385, size=48)
    kv = np.concatenate([dec, [4096 + 512, 4096 + 512]])
    n = np.concatenate([np.ones(48, np.int64), [512, 512]])
    b = Paged(torch, rng, kv, n)
    g = torch.Generator(device="cuda").manual_seed(6)
    # Slot mapping of the new tokens (positions kv_len - n .. kv_len - 1 of each sequence), PlanRegionWriter's rule.
    slots_h = []
    for i in range(b.batch):
        pages = b.kv_indices_h[b.kv_indptr_h[i]:b.kv_indptr_h[i + 1]].astype(np.int64)
        pos = np.arange(kv[i] - n[i], kv[i])
        slots_h.append(pages[pos // b.ps] * b.ps + pos % b.ps)
    slot_mapping = torch.from_numpy(np.concatenate(slots_h)).cuda()
    new_k = (torch.randn((b.tokens, b.hkv, b.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    new_v = (torch.randn((b.tokens, b.hkv, b.d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    cw = roost_amd.cache_write_params(new_k, new_v, b.k, b.v, slot_mapping, kv_heads=b.hkv, head_dim=b.d,
                                      page_size=b.ps)
    att = b.params(roost_amd)
    T, B = b.tokens, b.batch
    fused = torch.randn((T, 3 * H * D), generator=g, device="cuda").to(torch.bfloat16)
    gg = -torch.nn.functional.softplus(torch.randn((T, H), generator=g, device="cuda"))
    beta = torch.sigmoid(torch.randn((T, H), generator=g, device="cuda")).to(torch.bfloat16)
    pool = torch.randn((3 * B, H, D, D), generator=g, device="cuda") * 0.01
    out = torch.empty((T, H, D), dtype=torch.bfloat16, device="cuda")
    cu_h = b.q_indptr_h.copy()
    cu = torch.from_numpy(cu_h).cuda()
    reach = (T - 1) * 3 * H * D + H * D
    gdn = []
    for layer in range(3):
        sl = torch.arange(layer * B, (layer + 1) * B, dtype=torch.int32, device="cuda")
        gdn.append(roost_amd.gated_delta_rule_params(
            fused, fused, fused, gg, beta, out, pool, sl, cu, batch=B, tokens=T, q_stride=3 * H * D,
            k_stride=3 * H * D, v_stride=3 * H * D, q_len=reach, k_len=reach, v_len=reach, q_offset=0,
            k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h))
    e_cw = session.lib.entry(roost_amd.CACHE_WRITE_VARIANT)
    e_att = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    e_gdn = session.lib.entry(roost_amd.RECURRENT_VARIANT)
    ws_cw, _ = planned(session, e_cw, cw, "mixed-cw")
    ws_att, plan_ms = planned(session, e_att, att, "mixed-att")
    ws_gdn = []
    for layer in range(3):
        w, _ = planned(session, e_gdn, gdn[layer], f"mixed-gdn{layer}")
        ws_gdn.append(w)

    def step():
        session.run(e_cw, cw, ws_cw)
        session.run(e_att, att, ws_att)
        for layer in range(3):
            session.run(e_gdn, gdn[layer], ws_gdn[layer])

    settle(session, step)
    for _ in range(warmup):
        step()
    session.stream.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(session.stream)
    t_issue = time.perf_counter()
    for _ in range(steps):
        step()
    issue_ms = (time.perf_counter() - t_issue) * 1e3 / steps
    end.record(session.stream)
    end.synchronize()
    step_ms = start.elapsed_time(end) / steps
    cold_ms = time_cold(torch, session, FLUSH, step, 10) if FLUSH is not None else None
    parts = {
        "cache_write": time_runs(torch, session, e_cw, cw, ws_cw, steps, warmup),
        "attention": time_runs(torch, session, e_att, att, ws_att, steps, warmup),
        "gdn_layer": time_runs(torch, session, e_gdn, gdn[0], ws_gdn[0], steps, warmup),
    }
    # The gates folded into the GDN call (roost_amd_gdn_recurrent_gated_run) against the two calls it replaces (the
    # GatedDeltaRuleGates op writing g and beta from a Qwen3.5 [tokens, 64] b|a projection, then the recurrent variant):
    # not part of config 5's step, reported beside it.
    proj = (torch.randn((T, 64), generator=g, device="cuda") * 4).to(torch.bfloat16)
    a_log = torch.randn((H,), generator=g, device="cuda") * 0.5
    dt_bias = torch.randn((H,), generator=g, device="cuda")
    reach_g = (T - 1) * 64 + H
    gkw = dict(tokens=T, v_heads=H, a_stride=64, b_stride=64, a_len=reach_g, b_len=reach_g, a_offset=16, b_offset=0)
    gates_sep = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, gg, beta, **gkw)
    gates_fused = roost_amd.gated_delta_rule_gates_params(proj, proj, a_log, dt_bias, None, None, **gkw)
    e_gates = session.lib.entry(roost_amd.GATES_VARIANT)
    ws_gates, _ = planned(session, e_gates, gates_sep, "mixed-gates")

    def gates_then_gdn():
        session.run(e_gates, gates_sep, ws_gates)
        session.run(e_gdn, gdn[0], ws_gdn[0])

    parts["gates_then_gdn_layer"] = time_each(torch, session, gates_then_gdn, steps)
    parts["gdn_layer_gates_fused"] = time_each(
        torch, session, lambda: roost_amd.gdn_recurrent_gated(session, gdn[0], gates_fused, key="mixed-gated"), steps)
    # Qwen3.5's attention output gate (SigmoidMul on the attention output) folded into the attention call
    # (roost_amd_paged_attention_gated_run) against the two calls it replaces: not part of config 5's step either.
    out_gate = (torch.randn((T, b.hq * b.d), generator=g, device="cuda") * 2).to(torch.bfloat16)
    sm = roost_amd.sigmoid_mul_params(b.out, out_gate, b.out, rows=T, dim=b.hq * b.d)
    e_sm = session.lib.entry(roost_amd.SIGMOID_MUL_VARIANT)

    def attention_then_gate():
        session.run(e_att, att, ws_att)
        session.run(e_sm, sm, None)

    roost_amd.paged_attention_gated(session, att, sm, key="mixed-att-gated")
    ws_att_gated = session._ws[(e_att.variant_id, "mixed-att-gated")][3]

    def attention_gated():
        import ctypes as C

        st = session.lib.dll.roost_amd_paged_attention_gated_run(session.ctx, C.addressof(att), C.addressof(sm),
                                                               C.addressof(ws_att_gated), C.c_void_p(session.stream_handle))
        assert st == 0, session.lib.last_error()

    parts["attention_then_sigmoid_mul"] = time_each(torch, session, attention_then_gate, steps)
    parts["attention_gate_fused"] = time_each(torch, session, attention_gated, steps)
    # HBM floor of the step: K/V of every context token, the KV append, and per GDN layer the states read and
    # written once plus q, k, v, g, beta and o of every token.
    kv_bytes = int(kv.sum()) * b.hkv * b.d * 2 * 2 + 2 * T * b.hkv * b.d * 2 * 2
    gdn_bytes = 3 * (2 * B * H * D * D * 4 + T * (4 * H * D * 2 + H * 6))
    floor_ms = (kv_bytes + gdn_bytes) / (HBM_PEAK_GBS * 1e6)
    return {"workload": "BASELINE config 5: 48 decode ctx U(1024, 16384) + 2 x 512-token chunks on 4096 prefixes; "
                        "CacheWrite + PagedAttention + 3 GDN layers (recurrent variant)",
            "step_ms": step_ms, "cold_step_ms": cold_ms, "host_issue_ms": issue_ms, "breakdown_ms": parts,
            "attention_plan_ms": plan_ms,
            "hbm_floor_ms": floor_ms, "hbm_frac": floor_ms / step_ms, "context_tokens": int(kv.sum()),
            "tokens": T}


def bench_layer_ops(torch, roost_amd, session, steps, warmup):
    """The GDN layer's neighbour ops at Qwen3.5 shapes over config 4's 4 x 4096 tokens (HBM-bound; bytes are each op's
    reads and writes once): CausalConv1d over the [tokens, 6144] q/k/v projection (width 4, SiLU, bf16 state),
    GatedDeltaRuleGates (16 heads, a and b columns of a [tokens, 32] projection), GatedRmsNorm (16 x 128 per token,
    f32 weight), SigmoidMul (the attention output gate, 8 x 256 per token) and RecurrentStateCopy (16 GDN state slots of
    1 MiB)."""
    T, B, CH, H, D = 4 * 4096, 4, 6144, 16, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    bf = lambda *shape: torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16)  # noqa: E731
    res = {}

    def timed(name, entry_id, params, nbytes):
        entry = session.lib.entry(entry_id)
        session.launch(entry, params)
        ms = time_runs(torch, session, entry, params, None, steps, warmup)
        res[name] = {"ms": ms, "gb_s": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}
        if FLUSH is not None:
            cold = time_cold(torch, session, FLUSH, lambda: session.run(entry, params, None), 10)
            res[name].update(cold_ms=cold, cold_hbm_frac=nbytes / cold / 1e6 / HBM_PEAK_GBS)

    x, w = bf(T, CH), bf(CH, 4)
    y = torch.empty_like(x)
    st = bf(B, CH, 3)
    slots = torch.arange(B, dtype=torch.int32, device="cuda")
    cu = torch.arange(0, T + 1, 4096, dtype=torch.int32, device="cuda")
    p = roost_amd.causal_conv1d_params(x, w, None, y, st, slots, cu, batch=B, tokens=T, channels=CH, width=4, silu=True)
    timed("causal_conv1d", roost_amd.CAUSAL_CONV1D_VARIANT, p, 2 * T * CH * 2 + CH * 4 * 2 + 2 * B * CH * 3 * 2)
    ba = bf(T, 2 * H)
    a_log = torch.randn(H, generator=g, device="cuda")
    dt_bias = torch.randn(H, generator=g, device="cuda")
    gg = torch.empty((T, H), dtype=torch.float32, device="cuda")
    beta = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    reach = (T - 1) * 2 * H + H
    p = roost_amd.gated_delta_rule_gates_params(ba, ba, a_log, dt_bias, gg, beta, tokens=T, v_heads=H, a_stride=2 * H,
                                                b_stride=2 * H, a_len=reach, b_len=reach, a_offset=H, b_offset=0)
    timed("gates", roost_amd.GATES_VARIANT, p, T * H * (2 + 2 + 4 + 2))
    core, z = bf(T * H, D), bf(T * H, D)
    nw = torch.randn(D, generator=g, device="cuda")
    out = torch.empty_like(core)
    p = roost_amd.gated_rms_norm_params(core, z, nw, out, rows=T * H, dim=D, eps=1e-6)
    timed("gated_rms_norm", roost_amd.GATED_RMS_NORM_VARIANT, p, 3 * T * H * D * 2)
    attn, gate = bf(T, 8 * 256), bf(T, 8 * 256)
    o2 = torch.empty_like(attn)
    p = roost_amd.sigmoid_mul_params(attn, gate, o2, rows=T, dim=8 * 256)
    timed("sigmoid_mul", roost_amd.SIGMOID_MUL_VARIANT, p, 3 * T * 8 * 256 * 2)
    pool = torch.zeros((32, H * D * D), dtype=torch.float32, device="cuda")
    pairs = torch.tensor([[i, 16 + i] for i in range(16)], dtype=torch.int32, device="cuda").reshape(-1)
    p = roost_amd.recurrent_state_copy_params(pool, pairs, slot_bytes=H * D * D * 4, count=16)
    timed("recurrent_state_copy", roost_amd.STATE_COPY_VARIANT, p, 2 * 16 * H * D * D * 4)
    return res


def bench_attention_input(torch, roost_amd, session, steps, warmup):
    """The attention layer's input ops at the Qwen3.5 full-attention shape (8 q heads, 2 KV heads, head dim 256,
    16-token pages, theta 1e7): QkvQkNormRopeCacheWrite over a prefill of 8192 tokens and over a decode step of 64
    tokens, and the unfused QkNorm and Rope over the 8192 tokens. Bytes are each op's reads and writes once: the fused
    op reads the [q | k | v] rows and writes q plus the k and v cache rows."""
    HQ, HK, D, BS = 8, 2, 256, 16
    g = torch.Generator(device="cuda").manual_seed(11)
    bf = lambda *shape: torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16)  # noqa: E731
    res = {}

    def timed(name, entry_id, params, nbytes):
        entry = session.lib.entry(entry_id)
        session.launch(entry, params)
        ms = time_runs(torch, session, entry, params, None, steps, warmup)
        res[name] = {"ms": ms, "gb_s": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}

    qw, kw = bf(D) * 0.1 + 1, bf(D) * 0.1 + 1
    for name, T in (("qkv_prefill_8192", 8192), ("qkv_decode_64", 64)):
        qkv = bf(T, (HQ + 2 * HK) * D)
        q = torch.empty((T, HQ, D), dtype=torch.bfloat16, device="cuda")
        pages = (T + BS - 1) // BS + 1
        kc = torch.zeros((pages, BS, HK, D), dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros_like(kc)
        pos = torch.arange(T, dtype=torch.int32, device="cuda") + 4096
        slots = torch.randperm(pages * BS, generator=g, device="cuda")[:T].to(torch.int64)
        p = roost_amd.qkv_qk_norm_rope_cache_write_params(qkv, q, qw, kw, pos, kc, vc, slots, tokens=T, q_heads=HQ,
                                                          kv_heads=HK, head_dim=D, page_size=BS, eps=1e-6, theta=1e7)
        nbytes = T * (HQ + 2 * HK) * D * 2 + T * (HQ + 2 * HK) * D * 2 + T * 12
        timed(name, roost_amd.QKV_VARIANT, p, nbytes)
    T = 8192
    q, k = bf(T, HQ, D), bf(T, HK, D)
    pos = torch.arange(T, dtype=torch.int32, device="cuda")
    p = roost_amd.qk_norm_params(q, k, qw, kw, tokens=T, q_heads=HQ, kv_heads=HK, head_dim=D, eps=1e-6)
    timed("qk_norm_8192", roost_amd.QK_NORM_VARIANT, p, 2 * T * (HQ + HK) * D * 2)
    p = roost_amd.rope_params(q, k, pos, tokens=T, q_heads=HQ, kv_heads=HK, head_dim=D, theta=1e7, rotary_dim=64)
    timed("rope_partial64_8192", roost_amd.ROPE_VARIANT, p, 2 * T * (HQ + HK) * D * 2)
    return res


def bench_dense_vs_sdpa(torch, roost_amd, session, steps, warmup):
    """A dense-equivalent causal prefill (4 fresh sequences of 4096 tokens, 8 query / 2 KV heads, head dims 256 and
    128) through this library's paged kernels, beside torch's own scaled_dot_product_attention (the ROCm build's flash
    backend) on the same shape with contiguous K/V -- the platform's stock attention as a point of comparison."""
    import torch.nn.functional as F

    res = {}
    for d in (256, 128):
        rng = np.random.default_rng(1)
        b = Paged(torch, rng, [4096] * 4, [4096] * 4, d=d)
        entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
        p = b.params(roost_amd)
        ws, _ = planned(session, entry, p, f"bench-dense-{d}")
        ms = time_runs(torch, session, entry, p, ws, max(steps // 4, 3), 2)
        flops = b.prefill_flops()
        q = torch.randn(4, 8, 4096, d, device="cuda", dtype=torch.bfloat16) * 0.5
        k = torch.randn(4, 2, 4096, d, device="cuda", dtype=torch.bfloat16) * 0.5
        v = torch.randn(4, 2, 4096, d, device="cuda", dtype=torch.bfloat16) * 0.5
        sdpa = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)  # noqa: E731
        for _ in range(2):
            sdpa()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            sdpa()
        e1.record()
        torch.cuda.synchronize()
        sdpa_ms = e0.elapsed_time(e1) / 5
        res[f"head_dim_{d}"] = {"ms": ms, "tflops": flops / ms / 1e9, "frac": flops / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                                "torch_sdpa_ms": sdpa_ms, "torch_sdpa_tflops": flops / sdpa_ms / 1e9}
    return res


def _host_info():
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "threads_available": threads, "cpu_model": model}


def _timed(fn):
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def cpu_baselines(b: Paged, pb: Paged):
    """The CpuOps restatement (oracle/cpuops.c: double precision, one rounding per output) timed on this host on the
    same inputs as the GPU rows: one thread (CpuOps itself is single-threaded) and OpenMP over (sequence, head) on every
    available core. Decode config 2 runs in full; prefill config 3 and GDN config 4 run on stated subsets and are
    scaled by the exact work ratio (flops, or tokens for the token-serial GDN recurrence), labelled as extrapolated.
    Returns (host info, table, the headline baseline in the headline's unit)."""
    import torch

    import oracle

    info = _host_info()
    nthr = info["threads_available"]
    host = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    rows = {}
    # Decode, config 2 (whole batch).
    k, v, q = host(b.k), host(b.v), host(b.q)
    out = np.zeros_like(q)
    dec_bytes = b.decode_bytes()

    def decode(threads):
        oracle.paged_attention(q, out, k, v, b.q_indptr_h, b.kv_indptr_h, b.kv_indices_h, b.last_h, batch=b.batch,
                               tokens=b.tokens, q_heads=8, kv_heads=2, head_dim=256, page_size=16, bf16=True,
                               threads=threads)

    for name, threads in (("1_thread", 1), ("openmp", nthr)):
        secs = _timed(lambda: decode(threads))
        rows[f"decode_config2_{name}"] = {"threads": threads, "seconds": secs, "gb_s": dec_bytes / secs / 1e9,
                                          "sample": "all 64 sequences"}
    del k, v
    # Prefill, config 3: sequence subsets, scaled by flops.
    pk, pv, pq = host(pb.k), host(pb.v), host(pb.q)
    n, pre = pb.q_lens, pb.kv_lens - pb.q_lens
    seq_flops = 4 * 8 * 256 * (n * pre + n * (n + 1) / 2)
    total = float(seq_flops.sum())

    def prefill(seqs, threads):
        qi = np.concatenate([[0], np.cumsum(n[seqs])]).astype(np.int32)
        pages = [pb.kv_indices_h[pb.kv_indptr_h[i]:pb.kv_indptr_h[i + 1]] for i in seqs]
        ki = np.concatenate([[0], np.cumsum([len(x) for x in pages])]).astype(np.int32)
        qq = np.concatenate([pq[pb.q_indptr_h[i]:pb.q_indptr_h[i + 1]] for i in seqs])
        oo = np.zeros_like(qq)
        return _timed(lambda: oracle.paged_attention(
            qq, oo, pk, pv, qi, ki, np.concatenate(pages).astype(np.int32), pb.last_h[seqs].copy(),
            batch=len(seqs), tokens=int(qi[-1]), q_heads=8, kv_heads=2, head_dim=256, page_size=16, bf16=True,
            threads=threads))

    order = np.argsort(seq_flops)
    for name, seqs, threads in (("1_thread", order[:1], 1), ("openmp", order[:3], nthr)):
        part = float(seq_flops[seqs].sum())
        secs = prefill(list(seqs), threads)
        rows[f"prefill_config3_{name}"] = {
            "threads": threads, "seconds_for_sample": secs, "seconds_extrapolated": secs * total / part,
            "tflops": part / secs / 1e12, "sample": f"sequences {sorted(int(x) for x in seqs)} "
            f"({part / 1e9:.1f} of {total / 1e9:.1f} GFLOP), scaled by the flop ratio"}
    # GDN, config 4 (recurrent form, 4 x 4096 tokens): one sequence on one thread, all four on every core.
    rng = np.random.default_rng(4)
    H, D, T1 = 16, 128, 4096

    def gdn(nseq, threads):
        T = nseq * T1
        rows_ = lambda: bf16_bits(rng.standard_normal((T, H * D), dtype=np.float32))  # noqa: E731
        qg, kg, vg = rows_(), rows_(), rows_()
        gg = (-np.logaddexp(0.0, rng.standard_normal((T, H)))).astype(np.float32)
        bb = bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal((T, H)))))
        pool = (rng.standard_normal((nseq, H, D, D), dtype=np.float32) * 0.01).astype(np.float32)
        oo = np.zeros((T, H, D), np.uint16)
        cu = (np.arange(nseq + 1) * T1).astype(np.int32)
        return _timed(lambda: oracle.gated_delta_rule(
            qg, kg, vg, gg, bb, oo, pool, np.arange(nseq, dtype=np.int32), cu, batch=nseq, tokens=T, k_heads=H,
            v_heads=H, k_dim=D, v_dim=D, bf16=True, beta_bf16=True, threads=threads))

    gdn_flops = 4 * T1 * H * 6 * D * D  # the recurrence: 6 dk dv per token and head
    for name, nseq, threads in (("1_thread", 1, 1), ("openmp", 4, nthr)):
        secs = gdn(nseq, threads)
        rows[f"gdn_config4_{name}"] = {"threads": threads, "seconds_for_sample": secs,
                                       "seconds_extrapolated": secs * 4 / nseq,
                                       "gflops": gdn_flops * nseq / 4 / secs / 1e9,
                                       "sample": f"{nseq} of 4 sequences of 4096 tokens (scaled by tokens)"}
    r = rows["decode_config2_1_thread"]
    headline = {"value": r["gb_s"], "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"CpuOps restatement (oracle/cpuops.c, double, 1 thread) over the whole config-2 decode "
                          f"batch ({int(b.kv_lens.sum())} context tokens) in {r['seconds']:.2f} s on "
                          f"{info['cpu_model']}"}
    return info, rows, headline


def measured_traffic():
    """HBM bytes per decode run() as measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes, scaled by a 1 GiB copy
    (profiles/decode_config2_trace.md gives the commands); None when no measurement is committed."""
    f = ROOT / "profiles" / "decode_config2_traffic.json"
    if not f.exists():
        return None
    return int(json.loads(f.read_text())["traffic_bytes_per_run"])


def _rounded(d):
    return {k: (round(v, 5) if isinstance(v, float) else _rounded(v) if isinstance(v, dict) else v) for k, v in d.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds each timed call is run back to back before its timing (0 for profiler passes)")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill128", "dense", "gdn", "mixed", "layer", "attn_in"], default=None,
                    help="run one workload only and print its timing (for profiler passes); no JSON line")
    args = ap.parse_args()
    global SETTLE_S
    SETTLE_S = args.settle
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the attention + GDN path on a single MI355X "
              "(sharding is described in DESIGN.md, not launched).", file=sys.stderr)
        sys.exit(2)

    import torch

    import roost_amd

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    torch.cuda.set_device(0)
    session = roost_amd.OpSession(device=0)
    global FLUSH
    FLUSH = Flush(torch)
    if args.only is not None:
        fn = {"decode": bench_decode, "prefill": bench_prefill, "gdn": bench_gdn, "mixed": bench_mixed,
              "layer": bench_layer_ops, "attn_in": bench_attention_input,
              "prefill128": lambda *a: bench_prefill(*a, d=128), "dense": bench_dense_vs_sdpa}[args.only]
        res = fn(torch, roost_amd, session, args.steps, args.warmup)
        log(f"{args.only}: {res[1] if isinstance(res, tuple) else res} ms")
        session.close()
        return
    log("decode (config 2) ...")
    b, dec_ms, dec_plan_ms = bench_decode(torch, roost_amd, session, args.steps, args.warmup)
    dec_bytes = b.decode_bytes()
    dec_gbs = dec_bytes / dec_ms / 1e6
    log(f"  {dec_ms * 1e3:.1f} us/step, {dec_gbs:.0f} GB/s")
    log("prefill (config 3) ...")
    pb, pre_ms, pre_plan_ms = bench_prefill(torch, roost_amd, session, args.steps, args.warmup)
    pre_tflops = pb.prefill_flops() / pre_ms / 1e9
    log(f"  {pre_ms * 1e3:.1f} us/step, {pre_tflops:.0f} TFLOP/s")
    _, pre128_ms, _ = bench_prefill(torch, roost_amd, session, args.steps, args.warmup, d=128)
    pre128_flops = pb.prefill_flops() / 2
    log(f"  head dim 128: {pre128_ms * 1e3:.1f} us/step, {pre128_flops / pre128_ms / 1e9:.0f} TFLOP/s")
    dense = bench_dense_vs_sdpa(torch, roost_amd, session, args.steps, args.warmup)
    log(f"  dense 4 x 4096 vs torch SDPA: {json.dumps(_rounded(dense))}")
    log("gdn (config 4) ...")
    gdn = bench_gdn(torch, roost_amd, session, args.steps, args.warmup)
    log(f"  {json.dumps(gdn)}")
    log("GDN layer neighbour ops ...")
    layer = bench_layer_ops(torch, roost_amd, session, args.steps, args.warmup)
    log(f"  {json.dumps(layer)}")
    log("attention input ops ...")
    attn_in = bench_attention_input(torch, roost_amd, session, args.steps, args.warmup)
    log(f"  {json.dumps(attn_in)}")
    log("mixed hybrid step (config 5) ...")
    mixed = bench_mixed(torch, roost_amd, session, max(args.steps // 2, 3), max(args.warmup // 2, 1))
    log(f"  {json.dumps(mixed)}")
    cpu = cpu_host = cpu_rows = None
    if not args.skip_cpu:
        log("cpu baselines ...")
        cpu_host, cpu_rows, cpu = cpu_baselines(b, pb)
        log(f"  {cpu_host} {json.dumps(_rounded(cpu_rows))}")
    line = {
        "metric": METRIC,
        "value": round(dec_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 q/K/V, random disjoint page lists)",
        "config": {"workload": "BASELINE config 2: paged decode, Qwen3.5-0.8B full-attention shape",
                   "batch": 64, "ctx": "U(512, 8192)", "context_tokens": int(b.kv_lens.sum()), "q_heads": 8,
                   "kv_heads": 2, "head_dim": 256, "page_size": 16, "pool_pages": b.pool},
        "cold": {"ms_per_step": round(b.cold_ms, 5), "gb_s": round(dec_bytes / b.cold_ms / 1e6, 1),
                 "note": "median of 10 launches, each after reading a 512 MiB buffer (evicts the 256 MB MALL)"},
        "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "algorithmic_bytes": dec_bytes, "kernel": "DecodeKernel + DecodeMergeKernel (one run())"},
        "plan_ms": {"decode": round(dec_plan_ms, 3), "prefill": round(pre_plan_ms, 3)},
        "prefill": {"workload": "BASELINE config 3: 8 seqs, chunk U(256, 2048) on prefix U(0, 6144), causal",
                    "ms": round(pre_ms, 4), "tflops": round(pre_tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "frac": round(pre_tflops / MFMA_BF16_PEAK_TFLOPS, 4), "flops": pb.prefill_flops(),
                    "query_tokens": pb.tokens, "stat": "median of back-to-back launches, attention call only",
                    "append_plus_attention_ms": round(pb.append_ms, 4),
                    "append_plus_attention_tflops": round(pb.prefill_flops() / pb.append_ms / 1e9, 1),
                    "head_dim_128": {"ms": round(pre128_ms, 4), "tflops": round(pre128_flops / pre128_ms / 1e9, 1),
                                     "frac": round(pre128_flops / pre128_ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
                                     "note": "the same draw at head dim 128 (not a BASELINE config)"},
                    "dense_4x4096_vs_torch_sdpa": _rounded(dense)},
        "gdn": {k: _rounded(v) for k, v in gdn.items()},
        "mixed_step": _rounded(mixed),
        "gdn_layer_ops": {k: _rounded(v) for k, v in layer.items()},
        "attention_input_ops": {k: _rounded(v) for k, v in attn_in.items()},
        "cpu_baseline": cpu,
        "cpu_baselines": {"host": cpu_host, "rows": _rounded(cpu_rows) if cpu_rows else None},
    }
    session.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
