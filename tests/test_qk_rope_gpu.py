"""The attention layer's input ops on the GPU through the C ABI: QkNorm, Rope and the fused QkvQkNormRopeCacheWrite,
against the CpuOps oracle, and the fused op against the library's own unfused calls.

Tolerances: the library computes in fp32 and the oracle in double, each rounding every stored element once. A bf16
result may therefore differ by one rounding step of its own, plus, after Rope, the effect of a one-step difference in
its normalised input (which moves the result by at most one ulp of the row's largest element): |d| <= 2^-7 |ref| +
2^-7 max|row|, far inside BASELINE's 2e-2 / 1e-2 bar. f32 results: |d| <= 2e-6 max|row| (sincosf of the reduced angle
and rsqrt are good to a few fp32 ulps). Cache rows are the library's own k and v moved bit for bit, so the fused op
must equal QkNorm, Rope and CacheWrite called in order exactly (CpuOps.Fused.cs:37-95, FusedOpsTests.cs:48-97)."""
import numpy as np
import pytest

import cases
import oracle
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _vals(a, bf16):
    return oracle.bf16_to_f64(a) if bf16 else np.asarray(a, np.float64)


def assert_rows_close(got, want, bf16, head_dim, what):
    g, w = _vals(got, bf16), _vals(want, bf16)
    assert np.all(np.isfinite(g)), what
    rows_g, rows_w = g.reshape(-1, head_dim), w.reshape(-1, head_dim)
    rowmax = np.abs(rows_w).max(axis=1, keepdims=True)
    bound = (2.0 ** -7 * np.abs(rows_w) + 2.0 ** -7 * rowmax) if bf16 else 2e-6 * rowmax + 1e-30
    d = np.abs(rows_g - rows_w)
    bad = d > bound
    if bad.any():
        r, c = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} elements out of bound, e.g. row {r} col {c}: got {rows_g[r, c]!r} "
                             f"want {rows_w[r, c]!r}")


def _data(rng, n, bf16, scale=1.0, offset=0.0):
    x = (rng.standard_normal(n) * scale + offset).astype(np.float32)
    return cases.bf16_bits(x) if bf16 else x


@pytest.mark.parametrize("bf16,tokens,hq,hk,hd,q_stride,k_stride", [
    (True, 37, 8, 2, 256, 0, 0),        # Qwen3.5 attention heads
    (True, 9, 16, 4, 128, 0, 0),
    (False, 11, 8, 2, 256, 0, 0),
    (True, 5, 4, 2, 96, 0, 0),          # 12 chunks: 16 lanes per row, 4 idle
    (True, 6, 3, 1, 64, 2 * 3 * 64, 0), # q heads inside a wider row (q and its gate side by side)
    (False, 4, 2, 1, 8, 0, 24),
    (True, 3, 2, 2, 6, 0, 0),           # scalar path, odd rows
    (False, 2, 2, 1, 1000, 0, 0),       # scalar path, 16 elements per lane
    (True, 2, 1, 1, 1024, 0, 0),        # widest head: two 16-byte chunks per lane
])
def test_qk_norm(session, bf16, tokens, hq, hk, hd, q_stride, k_stride):
    rng = np.random.default_rng(hd + tokens)
    qs, ks = q_stride or hq * hd, k_stride or hk * hd
    q = _data(rng, (tokens - 1) * qs + hq * hd, bf16, 2.0)
    k = _data(rng, (tokens - 1) * ks + hk * hd, bf16, 2.0)
    qw, kw = _data(rng, hd, bf16, 0.1, 1.0), _data(rng, hd, bf16, 0.1, 1.0)
    want_q, want_k = q.copy(), k.copy()
    oracle.qk_norm(want_q, want_k, qw, kw, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, eps=1e-6,
                   q_stride=q_stride, k_stride=k_stride)
    dq, dk = to_dev(q, bf16), to_dev(k, bf16)
    roost_amd.qk_norm(session, dq, dk, to_dev(qw, bf16), to_dev(kw, bf16), tokens=tokens, q_heads=hq, kv_heads=hk,
                      head_dim=hd, eps=1e-6, q_stride=q_stride, k_stride=k_stride)
    gq, gk = from_dev(dq, bf16), from_dev(dk, bf16)
    # Elements between the head rows of a strided layout are left exactly as they were.
    for got, want, orig, stride, heads in ((gq, want_q, q, qs, hq), (gk, want_k, k, ks, hk)):
        mask = np.zeros(got.size, bool)
        for t in range(tokens):
            mask[t * stride:t * stride + heads * hd] = True
        assert np.array_equal(got[~mask], orig[~mask])
        assert_rows_close(got[mask], want[mask], bf16, hd, "qk norm")


@pytest.mark.parametrize("bf16,tokens,hq,hk,hd,rot,interleaved,llama3,max_pos", [
    (True, 33, 8, 2, 256, 64, False, None, 262144),   # Qwen3.5: a quarter of the head rotated, long positions
    (True, 17, 8, 2, 256, 0, False, None, 4096),
    (False, 9, 4, 2, 128, 0, True, None, 70000),
    (True, 7, 4, 1, 128, 0, False, (8.0, 1.0, 4.0, 8192), 131072),
    (False, 5, 2, 2, 64, 32, True, (32.0, 1.0, 4.0, 8192), 1000),
    (True, 4, 2, 1, 10, 6, False, None, 100),          # scalar path, partial width
    (True, 6, 4, 2, 64, 24, False, None, 9000),        # vector rows, NeoX halves not whole chunks: per-element pairs
    (True, 6, 4, 2, 64, 20, True, None, 9000),         # vector rows, interleaved width not a whole chunk
    (False, 3, 1, 1, 1000, 0, False, None, 50000),     # scalar path, 16 elements per lane
])
def test_rope(session, bf16, tokens, hq, hk, hd, rot, interleaved, llama3, max_pos):
    rng = np.random.default_rng(hd * 7 + tokens)
    q, k = _data(rng, tokens * hq * hd, bf16), _data(rng, tokens * hk * hd, bf16)
    pos = rng.integers(0, max_pos, tokens).astype(np.int32)
    pos[0] = 0
    theta = 1e6 if llama3 is None else 5e5
    want_q, want_k = q.copy(), k.copy()
    oracle.rope(want_q, want_k, pos, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, theta=theta,
                rotary_dim=rot, interleaved=interleaved, llama3=llama3)
    dq, dk = to_dev(q, bf16), to_dev(k, bf16)
    roost_amd.rope(session, dq, dk, to_dev(pos), tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, theta=theta,
                   rotary_dim=rot, interleaved=interleaved, llama3=llama3)
    gq, gk = from_dev(dq, bf16), from_dev(dk, bf16)
    assert_rows_close(gq, want_q, bf16, hd, "rope q")
    assert_rows_close(gk, want_k, bf16, hd, "rope k")
    # Position 0 is the identity, and dims at and beyond the rotary width are untouched, bit for bit.
    assert np.array_equal(gq[:hq * hd], q[:hq * hd])
    r = rot or hd
    assert np.array_equal(gq.reshape(-1, hd)[:, r:], q.reshape(-1, hd)[:, r:])


def _fused_case(rng, tokens, hq, hk, hd, bs, blocks, bf16):
    row = (hq + 2 * hk) * hd
    qkv = _data(rng, tokens * row, bf16, 1.5)
    qw, kw = _data(rng, hd, bf16, 0.1, 1.0), _data(rng, hd, bf16, 0.1, 1.0)
    pos = rng.integers(0, 40000, tokens).astype(np.int32)
    # Distinct slots, one negative and one beyond the pool (both write no cache row).
    slots = rng.permutation(blocks * bs)[:tokens].astype(np.int64)
    slots[1 % tokens] = -1
    if tokens > 2:
        slots[2] = blocks * bs + 5
    return qkv, qw, kw, pos, slots


@pytest.mark.parametrize("bf16,kv_f32,tokens,hq,hk,hd,bs", [
    (True, False, 41, 8, 2, 256, 16),   # Qwen3.5 full-attention layer shape
    (True, True, 9, 4, 2, 128, 4),      # bf16 activations into f32 pages
    (False, False, 13, 4, 1, 64, 8),
    (True, False, 5, 4, 2, 8, 4),       # the reference's FusedOpsTests shape
    (True, False, 3, 2, 1, 6, 2),       # scalar path
])
def test_fused_qkv_matches_oracle_and_unfused_calls(session, bf16, kv_f32, tokens, hq, hk, hd, bs):
    import torch

    rng = np.random.default_rng(tokens * 31 + hd)
    blocks = (tokens + bs - 1) // bs + 3
    qkv, qw, kw, pos, slots = _fused_case(rng, tokens, hq, hk, hd, bs, blocks, bf16)
    kv_bits = bf16 and not kv_f32
    pool = blocks * bs * hk * hd
    fill = cases.bf16_bits(np.full(pool, 0.25, np.float32)) if kv_bits else np.full(pool, 0.25, np.float32)
    want_q = np.zeros(tokens * hq * hd, qkv.dtype)
    want_kc, want_vc = fill.copy(), fill.copy()
    ok = (slots >= 0) & (slots < blocks * bs)
    oracle.qkv_qk_norm_rope_cache_write(qkv, want_q, qw, kw, pos, want_kc, want_vc, np.where(ok, slots, -1),
                                        tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, page_size=bs, eps=1e-6,
                                        theta=1e6)
    d_qkv = to_dev(qkv, bf16)
    d_q = torch.full((tokens * hq * hd,), float("nan"), device="cuda",
                     dtype=torch.bfloat16 if bf16 else torch.float32)
    d_kc, d_vc = to_dev(fill, kv_bits), to_dev(fill, kv_bits)
    d_pos, d_slots = to_dev(pos), to_dev(slots)
    d_qw, d_kw = to_dev(qw, bf16), to_dev(kw, bf16)
    roost_amd.qkv_qk_norm_rope_cache_write(session, d_qkv, d_q, d_qw, d_kw, d_pos, d_kc, d_vc, d_slots, tokens=tokens,
                                           q_heads=hq, kv_heads=hk, head_dim=hd, page_size=bs, eps=1e-6, theta=1e6)
    got_q, got_kc, got_vc = from_dev(d_q, bf16), from_dev(d_kc, kv_bits), from_dev(d_vc, kv_bits)
    assert np.array_equal(from_dev(d_qkv, bf16), qkv), "qkv must be left as it was"
    assert_rows_close(got_q, want_q, bf16, hd, "fused q")
    # v rows are moved bit for bit; rows the slots do not name keep the fill.
    assert np.array_equal(got_vc, want_vc)
    assert_rows_close(got_kc, want_kc, bf16 and not kv_f32, hd, "fused k cache")
    written = np.zeros(blocks * bs, bool)
    written[slots[ok]] = True
    kc_rows = got_kc.reshape(blocks * bs, -1)
    assert np.array_equal(kc_rows[~written], fill.reshape(blocks * bs, -1)[~written])
    if kv_f32:
        return  # CacheWrite moves equal types only; the widening is checked against the oracle above
    # The same call as QkNorm, Rope and CacheWrite in order, on the GPU: bit-identical q and pools.
    q = torch.empty_like(d_q)
    k = torch.empty((tokens * hk * hd,), device="cuda", dtype=q.dtype)
    v = torch.empty_like(k)
    rows = d_qkv.view(tokens, -1)
    q.view(tokens, -1).copy_(rows[:, :hq * hd])
    k.view(tokens, -1).copy_(rows[:, hq * hd:(hq + hk) * hd])
    v.view(tokens, -1).copy_(rows[:, (hq + hk) * hd:])
    roost_amd.qk_norm(session, q, k, d_qw, d_kw, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, eps=1e-6)
    roost_amd.rope(session, q, k, d_pos, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, theta=1e6)
    kc2, vc2 = to_dev(fill, kv_bits), to_dev(fill, kv_bits)
    roost_amd.cache_write(session, k.view(tokens, hk, hd), v.view(tokens, hk, hd), kc2, vc2, d_slots, kv_heads=hk,
                          head_dim=hd, page_size=bs)
    assert np.array_equal(from_dev(q, bf16), got_q)
    assert np.array_equal(from_dev(kc2, kv_bits), got_kc)
    assert np.array_equal(from_dev(vc2, kv_bits), got_vc)


def test_fused_qkv_replays_in_a_graph(session):  # the fixture skips without a GPU; the graph gets its own session
    """GRAPH_CAPTURABLE: one captured call replayed three times, with eager work between the replays, gives the eager
    result bit for bit every time."""
    import torch

    rng = np.random.default_rng(77)
    tokens, hq, hk, hd, bs, blocks = 24, 8, 2, 256, 16, 6
    qkv, qw, kw, pos, slots = _fused_case(rng, tokens, hq, hk, hd, bs, blocks, True)
    pool = blocks * bs * hk * hd
    stream = torch.cuda.Stream()
    session = roost_amd.OpSession(session.lib, stream=stream)
    try:
        d_qkv, d_qw, d_kw, d_pos, d_slots = to_dev(qkv, True), to_dev(qw, True), to_dev(kw, True), to_dev(pos), \
            to_dev(slots)
        q = torch.zeros(tokens * hq * hd, device="cuda", dtype=torch.bfloat16)
        kc = torch.zeros(pool, device="cuda", dtype=torch.bfloat16)
        vc = torch.zeros(pool, device="cuda", dtype=torch.bfloat16)
        entry = session.lib.entry(roost_amd.QKV_VARIANT)
        p = roost_amd.qkv_qk_norm_rope_cache_write_params(d_qkv, q, d_qw, d_kw, d_pos, kc, vc, d_slots, tokens=tokens,
                                                          q_heads=hq, kv_heads=hk, head_dim=hd, page_size=bs,
                                                          eps=1e-6, theta=1e6)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            session.run(entry, p, None)
        stream.synchronize()
        want = (q.clone(), kc.clone(), vc.clone())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            session.run(entry, p, None)
        for replay in range(3):
            with torch.cuda.stream(stream):  # the replay too: replay() launches on the current stream
                q.fill_(float("nan"))
                kc.zero_()
                vc.zero_()
                graph.replay()
            stream.synchronize()
            for got, exp in zip((q, kc, vc), want):
                assert torch.equal(got.view(torch.int16), exp.view(torch.int16)), f"replay {replay}"
    finally:
        session.close()


def test_refusals(session):
    import torch

    x = torch.zeros(4096, device="cuda", dtype=torch.bfloat16)
    pos = torch.zeros(8, device="cuda", dtype=torch.int32)
    sl = torch.zeros(8, device="cuda", dtype=torch.int64)
    def status(variant, p):
        return session.run_raw(session.lib.entry(variant), p, None)

    p = roost_amd.qk_norm_params(x, x, x, x, tokens=2, q_heads=0, kv_heads=1, head_dim=64, eps=1e-6)
    assert status(roost_amd.QK_NORM_VARIANT, p) == abi.INVALID_ARGUMENT
    p = roost_amd.qk_norm_params(x, x, x, x, tokens=2, q_heads=2, kv_heads=1, head_dim=64, eps=1e-6, q_stride=64)
    assert status(roost_amd.QK_NORM_VARIANT, p) == abi.INVALID_ARGUMENT
    f16 = torch.zeros(64, device="cuda", dtype=torch.float16)
    p = roost_amd.qk_norm_params(f16, f16, f16, f16, tokens=1, q_heads=1, kv_heads=1, head_dim=16, eps=1e-6)
    assert status(roost_amd.QK_NORM_VARIANT, p) == abi.UNSUPPORTED
    p = roost_amd.rope_params(x, x, pos, tokens=2, q_heads=1, kv_heads=1, head_dim=64, theta=1e4, rotary_dim=63)
    assert status(roost_amd.ROPE_VARIANT, p) == abi.INVALID_ARGUMENT
    p = roost_amd.rope_params(x, x, pos, tokens=2, q_heads=1, kv_heads=1, head_dim=64, theta=0.0)
    assert status(roost_amd.ROPE_VARIANT, p) == abi.INVALID_ARGUMENT
    p = roost_amd.rope_params(x, x, pos, tokens=2, q_heads=1, kv_heads=1, head_dim=64, theta=1e4,
                              llama3=(8.0, 4.0, 1.0, 8192))
    assert status(roost_amd.ROPE_VARIANT, p) == abi.INVALID_ARGUMENT
    p = roost_amd.rope_params(x, x, pos, tokens=100, q_heads=1, kv_heads=1, head_dim=64, theta=1e4)
    assert status(roost_amd.ROPE_VARIANT, p) == abi.INVALID_ARGUMENT  # q and k too short
    # The fused op: an undersized qkv is refused before anything is written (FusedOpsTests.cs:99-113).
    q = torch.full((64,), 3.0, device="cuda", dtype=torch.bfloat16)
    kc = torch.zeros(4096, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros(4096, device="cuda", dtype=torch.bfloat16)
    small = torch.zeros(11, device="cuda", dtype=torch.bfloat16)
    p = roost_amd.qkv_qk_norm_rope_cache_write_params(small, q, x, x, pos, kc, vc, sl, tokens=2, q_heads=1, kv_heads=1,
                                                      head_dim=2, page_size=2, eps=1e-6, theta=1e4)
    assert status(roost_amd.QKV_VARIANT, p) == abi.INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert bool((q == 3.0).all())
    # Cache of another type than the activations (other than f32 under bf16) is not built.
    kc16 = torch.zeros(4096, device="cuda", dtype=torch.float16)
    p = roost_amd.qkv_qk_norm_rope_cache_write_params(x, q, x, x, pos, kc16, kc16, sl, tokens=2, q_heads=1,
                                                      kv_heads=1, head_dim=8, page_size=2, eps=1e-6, theta=1e4)
    assert status(roost_amd.QKV_VARIANT, p) == abi.UNSUPPORTED
    # q may not overlap qkv.
    p = roost_amd.qkv_qk_norm_rope_cache_write_params(x, x, x, x, pos, kc, vc, sl, tokens=2, q_heads=1, kv_heads=1,
                                                      head_dim=8, page_size=2, eps=1e-6, theta=1e4)
    assert status(roost_amd.QKV_VARIANT, p) == abi.INVALID_ARGUMENT
