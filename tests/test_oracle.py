"""Pins the CpuOps oracle (oracle/cpuops.c) before any GPU result is compared with it.

Which check pins which oracle function:
  to_bf16          -- bit patterns: ties to even, round-to-odd double rounding, NaN -> 0x7FC0, overflow -> inf
                      (CpuElements.cs:128-160), and exhaustive agreement with float32 RNE for float32 inputs.
  paged_attention  -- the reference's hand cases (AttentionTests.cs:135-228: two-key 7.0, bf16 mean [2, 3], window and
                      no-pages zeros, out-of-range last page length refused), the reference's independent dense
                      three-pass formulation over its 9 parameter rows at 1e-12 (AttentionTests.cs:8-133, restated
                      here in numpy), and torch's float64 scaled_dot_product_attention on de-paged K/V.
  cache_write      -- the hand case BasicOpsTests.cs:202-232 (NHD and HND) and a scatter/gather round trip.
  gated_delta_rule -- the scalar hand case HybridTests.cs:7-24 (o = [1, 3], S = 1), the matrix formulation
                      S' = (I - b k k^T) e^g S + b k v^T with grouped heads and slots (HybridTests.cs:32-172), two calls
                      = one call and token-by-token decode (HybridTests.cs:174-220), scale 0 = 1/sqrt(k_dim), and
                      strided views = contiguous copies (GatedDeltaRuleViewTests.cs).
  qk_norm          -- the hand case BasicOpsTests.cs:35-46 (two query heads, one key head, each with its own weight),
                      per-token strides = contiguous copies, and the mean square of a unit-weight row being 1.
  rope             -- the hand cases BasicOpsTests.cs:65-116 (NeoX halves, interleaved pairs, partial rotary width,
                      position 0, Llama 3 low-frequency scaling at 1e-11), transformers 5.20.1's Llama 3 cos/sin rows
                      (the reference fixture, RopeScalingTests.cs:105-127), and the rotation laws: pair norms kept,
                      rope(p1) then rope(p2) = rope(p1 + p2).
  plan_region      -- the closed form slot = block[pos / bs] * bs + pos % bs and the indptr prefix sums
                      (PlanRegionWriter.cs:19-64) on hand-written plans.
"""
import math

import numpy as np
import pytest

import cases
import oracle


# ---- elements ----------------------------------------------------------------------------------------------------------

def test_bf16_rounding_bit_patterns():
    assert oracle.to_bf16(1.0) == 0x3F80
    # Ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7.
    assert oracle.to_bf16(1.0 + 2 ** -8) == 0x3F80
    assert oracle.to_bf16(1.0 + 3 * 2 ** -8) == 0x3F82
    # Just above the tie rounds up: double rounding through float would lose this (1 + 2^-8 + 2^-40 -> float tie).
    assert oracle.to_bf16(1.0 + 2 ** -8 + 2 ** -40) == 0x3F81
    assert oracle.to_bf16(float("nan")) == 0x7FC0
    assert oracle.to_bf16(float("inf")) == 0x7F80 and oracle.to_bf16(float("-inf")) == 0xFF80
    assert oracle.to_bf16(3.5e38) == 0x7F80  # beyond the largest finite bf16
    assert oracle.to_bf16(-0.0) == 0x8000


def test_bf16_rounding_agrees_with_float32_rne():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000)
    x = x.astype(np.float32)
    want = oracle.f32_to_bf16_rne(x)
    got = oracle.to_bf16(x.astype(np.float64))
    assert np.array_equal(got, want)


# ---- attention ---------------------------------------------------------------------------------------------------------

def attention_f64(q, k_pool, v_pool, q_indptr, kv_indptr, kv_indices, last, *, batch, tokens, hq, hkv, hd, bs, hnd,
                  scale=0.0, cap=0.0, window=-1, causal=True):
    out = np.zeros((tokens, hq, hd))
    oracle.paged_attention(np.ascontiguousarray(q, np.float64), out, np.ascontiguousarray(k_pool, np.float64),
                           np.ascontiguousarray(v_pool, np.float64), np.asarray(q_indptr, np.int32),
                           np.asarray(kv_indptr, np.int32), np.asarray(kv_indices, np.int32),
                           np.asarray(last, np.int32), batch=batch, tokens=tokens, q_heads=hq, kv_heads=hkv,
                           head_dim=hd, page_size=bs, hnd=hnd, scale=scale, soft_cap=cap, window_left=window,
                           causal=causal, threads=1)
    return out


def test_two_key_hand_case():
    # One head of width 1, scale 1: scores 0 and ln 3 -> weights 1/4, 3/4 -> 0.25 * 4 + 0.75 * 8 = 7.
    out = attention_f64([[[1.0]]], [0.0, math.log(3)], [4.0, 8.0], [0, 1], [0, 1], [0], [2], batch=1, tokens=1, hq=1,
                        hkv=1, hd=1, bs=2, hnd=False, scale=1.0)
    assert abs(out[0, 0, 0] - 7.0) < 1e-13


def test_bf16_cache_mean_hand_case():
    q = cases.bf16_bits(np.array([[[1.0, 0.0]]], np.float32))
    k = cases.bf16_bits(np.array([1, 0, 1, 0], np.float32))
    v = cases.bf16_bits(np.array([1, 2, 3, 4], np.float32))
    out = np.zeros_like(q)
    oracle.paged_attention(q, out, k, v, np.array([0, 1], np.int32), np.array([0, 1], np.int32),
                           np.array([0], np.int32), np.array([2], np.int32), batch=1, tokens=1, q_heads=1, kv_heads=1,
                           head_dim=2, page_size=2, bf16=True)
    assert list(cases.bf16_values(out).ravel()) == [2.0, 3.0]


def test_window_of_one_and_no_pages_give_expected():
    out = attention_f64([[[1.0]]], [1.0, 1.0], [5.0, 5.0], [0, 1], [0, 1], [0], [2], batch=1, tokens=1, hq=1, hkv=1,
                        hd=1, bs=2, hnd=False, window=1)
    assert abs(out[0, 0, 0] - 5.0) < 1e-13
    out = attention_f64([[[1.0]]], [1.0, 1.0], [5.0, 5.0], [0, 1], [0, 0], [0], [2], batch=1, tokens=1, hq=1, hkv=1,
                        hd=1, bs=2, hnd=False, causal=False)
    assert out[0, 0, 0] == 0.0


@pytest.mark.parametrize("last", [3, 0, -1])
def test_out_of_range_last_page_length_is_refused_before_writing(last):
    out = np.full((1, 1, 1), 99.0)
    with pytest.raises(oracle.OracleError):
        oracle.paged_attention(np.ones((1, 1, 1)), out, np.ones(2), np.full(2, 5.0), np.array([0, 1], np.int32),
                               np.array([0, 1], np.int32), np.array([0], np.int32), np.array([last], np.int32),
                               batch=1, tokens=1, q_heads=1, kv_heads=1, head_dim=1, page_size=2)
    assert out[0, 0, 0] == 99.0
    with pytest.raises(oracle.OracleError):  # WindowLeft 0 is an unbound field
        oracle.paged_attention(np.ones((1, 1, 1)), out, np.ones(2), np.full(2, 5.0), np.array([0, 1], np.int32),
                               np.array([0, 1], np.int32), np.array([0], np.int32), np.array([2], np.int32),
                               batch=1, tokens=1, q_heads=1, kv_heads=1, head_dim=1, page_size=2, window_left=0)


def dense_reference(q, k, v, q_lens, hq, hkv, hd, causal, window, scale, cap):
    """Three-pass softmax over dense per-sequence K/V, no online rescaling (the reference's independent formulation,
    AttentionTests.cs:8-56)."""
    outs, qi = [], 0
    for b, n in enumerate(q_lens):
        kv_len = k[b].shape[0]
        for i in range(n):
            qpos = kv_len - n + i
            for h in range(hq):
                kvh = h // (hq // hkv)
                ok = np.array([(not causal or j <= qpos) and (window < 0 or j >= qpos - window) for j in range(kv_len)])
                s = k[b][:, kvh * hd:(kvh + 1) * hd] @ q[qi][h * hd:(h + 1) * hd] * scale
                if cap != 0:
                    s = cap * np.tanh(s / cap)
                mx = s[ok].max() if ok.any() else 0.0
                z = np.exp(s[ok] - mx).sum()
                w = np.where(ok, np.exp(s - mx) / z, 0.0)
                outs.append(w @ v[b][:, kvh * hd:(kvh + 1) * hd])
            qi += 1
    return np.array(outs).ravel()


ROWS = [(False, False, -1, 0.0, 0.0), (True, False, -1, 0.0, 0.0), (False, True, -1, 0.0, 0.0),
        (True, True, -1, 0.0, 0.0), (False, True, 3, 0.0, 0.0), (True, True, 3, 0.0, 0.0),
        (False, True, -1, 0.0, 5.0), (True, True, 2, 0.37, 3.0), (False, False, 4, 0.0, 0.0)]


@pytest.mark.parametrize("hnd,causal,window,scale_arg,cap", ROWS)
def test_matches_dense_three_pass_through_shuffled_blocks(hnd, causal, window, scale_arg, cap):
    hq, hkv, hd, bs = 4, 2, 8, 4
    kv_lens, q_lens = [7, 10], [3, 1]
    rng = np.random.default_rng(1234)
    q = [rng.uniform(-1, 1, hq * hd) for _ in range(sum(q_lens))]
    k = [rng.uniform(-1, 1, (n, hkv * hd)) for n in kv_lens]
    v = [rng.uniform(-1, 1, (n, hkv * hd)) for n in kv_lens]
    table = [[5, 2], [7, 0, 3]]
    kp = np.zeros(8 * bs * hkv * hd)
    vp = np.zeros_like(kp)
    for b in range(2):
        for j in range(kv_lens[b]):
            blk, off = table[b][j // bs], j % bs
            for h in range(hkv):
                for d in range(hd):
                    idx = (((blk * hkv + h) * bs + off) * hd + d) if hnd else (((blk * bs + off) * hkv + h) * hd + d)
                    kp[idx] = k[b][j, h * hd + d]
                    vp[idx] = v[b][j, h * hd + d]
    out = attention_f64(np.array(q).reshape(4, hq, hd), kp, vp, [0, 3, 4], [0, 2, 5], [5, 2, 7, 0, 3], [3, 2],
                        batch=2, tokens=4, hq=hq, hkv=hkv, hd=hd, bs=bs, hnd=hnd, scale=scale_arg, cap=cap,
                        window=window, causal=causal)
    scale = 1.0 / math.sqrt(hd) if scale_arg == 0 else float(np.float32(scale_arg))
    want = dense_reference(q, k, v, q_lens, hq, hkv, hd, causal, window, scale, float(np.float32(cap)))
    assert np.max(np.abs(out.ravel() - want)) < 1e-12


def test_matches_torch_float64_sdpa():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    b = cases.make_paged_batch(rng, [37, 100], [5, 100], page_size=16, bf16=False, d=32)
    q = b.q.astype(np.float64)
    kp = b.k_cache.astype(np.float64)
    vp = b.v_cache.astype(np.float64)
    out = attention_f64(q, kp, vp, b.q_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, batch=2,
                        tokens=b.tokens, hq=8, hkv=2, hd=32, bs=16, hnd=False)
    for s in range(2):
        pages = b.kv_indices[b.kv_indptr[s]:b.kv_indptr[s + 1]]
        k = torch.from_numpy(kp[pages].reshape(-1, 2, 32)[: b.kv_lens[s]]).repeat_interleave(4, dim=1)
        v = torch.from_numpy(vp[pages].reshape(-1, 2, 32)[: b.kv_lens[s]]).repeat_interleave(4, dim=1)
        qq = torch.from_numpy(q[b.q_indptr[s]:b.q_indptr[s + 1]])
        n, kl = qq.shape[0], k.shape[0]
        mask = torch.arange(kl)[None, :] <= torch.arange(kl - n, kl)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qq.transpose(0, 1), k.transpose(0, 1),
                                                               v.transpose(0, 1), attn_mask=mask)
        assert np.max(np.abs(ref.transpose(0, 1).numpy() - out[b.q_indptr[s]:b.q_indptr[s + 1]])) < 1e-12


# ---- cache write -------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("hnd", [False, True])
def test_cache_write_hand_case(hnd):
    k = cases.bf16_bits(np.arange(1, 13, dtype=np.float32))
    v = cases.bf16_bits(-np.arange(1, 13, dtype=np.float32))
    kc = np.zeros(16, np.uint16)
    vc = np.zeros(16, np.uint16)
    oracle.cache_write(k, v, kc, vc, np.array([3, -1, 0], np.int64), tokens=3, kv_heads=2, head_dim=2, page_size=2,
                       hnd=hnd, bf16=True)
    expected = np.zeros(16)
    for h in range(2):
        for d in range(2):
            idx = (lambda blk, off: ((blk * 2 + h) * 2 + off) * 2 + d) if hnd else \
                (lambda blk, off: ((blk * 2 + off) * 2 + h) * 2 + d)
            expected[idx(1, 1)] = h * 2 + d + 1
            expected[idx(0, 0)] = 8 + h * 2 + d + 1
    assert np.array_equal(cases.bf16_values(kc), expected)
    assert np.array_equal(cases.bf16_values(vc), -expected)


def test_cache_write_round_trip_and_skips():
    rng = np.random.default_rng(2)
    tokens, hkv, d, ps, pages = 50, 2, 8, 4, 20
    k = rng.integers(0, 65536, (tokens, hkv, d), dtype=np.uint16)
    kc = np.full((pages, ps, hkv, d), 0xABAB, np.uint16)
    slots = rng.permutation(pages * ps)[:tokens].astype(np.int64)
    slots[::5] = -1
    oracle.cache_write(k, k, kc, kc.copy(), slots, tokens=tokens, kv_heads=hkv, head_dim=d, page_size=ps, bf16=True)
    flat = kc.reshape(pages * ps, hkv, d)
    for t in range(tokens):
        if slots[t] >= 0:
            assert np.array_equal(flat[slots[t]], k[t])
    untouched = np.setdiff1d(np.arange(pages * ps), slots[slots >= 0])
    assert np.all(flat[untouched] == 0xABAB)


# ---- gated delta rule --------------------------------------------------------------------------------------------------

def gdn_f64(q, k, v, g, beta, state, slots, cu, *, kh, vh, kd, vd, scale, init, l2, tokens, batch):
    out = np.zeros((tokens, vh, vd))
    oracle.gated_delta_rule(np.ascontiguousarray(q, np.float64), np.ascontiguousarray(k, np.float64),
                            np.ascontiguousarray(v, np.float64), np.ascontiguousarray(g, np.float64),
                            np.ascontiguousarray(beta, np.float64), out, state, np.asarray(slots, np.int32),
                            np.asarray(cu, np.int32), batch=batch, tokens=tokens, k_heads=kh, v_heads=vh, k_dim=kd,
                            v_dim=vd, use_initial_state=init, l2_norm_qk=l2, scale=scale, threads=1)
    return out


def test_gdn_scalar_hand_case():
    # t0: S = 0, d = 0.5 * (2 - 0) = 1, S = 1, o = 1.  t1: S = 2, d = 1 * (1 - 2) = -1, S = 1, o = 3.
    state = np.array([123.0], np.float32)
    out = gdn_f64([1, 3], [1, 1], [2, 1], [0, math.log(2)], [0.5, 1], state, [0], [0, 2], kh=1, vh=1, kd=1, vd=1,
                  scale=1.0, init=False, l2=False, tokens=2, batch=1)
    assert np.max(np.abs(out.ravel() - [1.0, 3.0])) < 1e-14
    assert state[0] == 1.0


def matrix_form(q, k, v, g, beta, s0, scale, l2):
    s = s0.copy()
    outs = []
    for t in range(len(q)):
        qt, kt = np.array(q[t]), np.array(k[t])
        if l2:
            qt = qt / math.sqrt((qt ** 2).sum() + 1e-6)
            kt = kt / math.sqrt((kt ** 2).sum() + 1e-6)
        s = (np.eye(len(kt)) - beta[t] * np.outer(kt, kt)) @ (math.exp(g[t]) * s) + beta[t] * np.outer(kt, v[t])
        outs.append(s.T @ (qt * scale))
    return np.array(outs), s


@pytest.mark.parametrize("l2", [False, True])
def test_gdn_matches_matrix_formulation_with_grouped_heads_and_slots(l2):
    kh, vh, kd, vd = 2, 4, 3, 2
    rng = np.random.default_rng(77)
    lens = [5, 3]
    tokens = sum(lens)
    q = rng.uniform(-1, 1, (tokens, kh, kd))
    k = rng.uniform(-1, 1, (tokens, kh, kd))
    v = rng.uniform(-1, 1, (tokens, vh, vd))
    g = -rng.uniform(0, 1, (tokens, vh))
    beta = rng.uniform(0, 1, (tokens, vh))
    pool = rng.uniform(-1, 1, (4, vh, kd, vd)).astype(np.float32)
    before = pool.copy()
    scale = float(np.float32(0.7))
    out = gdn_f64(q, k, v, g, beta, pool, [3, 1], [0, 5, 8], kh=kh, vh=vh, kd=kd, vd=vd, scale=0.7, init=True, l2=l2,
                  tokens=tokens, batch=2)
    t0 = 0
    for b, slot in enumerate([3, 1]):
        for h in range(vh):
            khd = h // (vh // kh)
            sl = slice(t0, t0 + lens[b])
            exp_o, s_end = matrix_form(q[sl, khd], k[sl, khd], v[sl, h], g[sl, h], beta[sl, h],
                                       before[slot, h].astype(np.float64), scale, l2)
            assert np.max(np.abs(out[sl, h] - exp_o)) < 1e-12
            assert np.max(np.abs(pool[slot, h] - s_end)) < 1e-6
        t0 += lens[b]
    assert np.array_equal(pool[0], before[0]) and np.array_equal(pool[2], before[2])


def test_gdn_two_calls_equal_one_call_and_token_decode():
    kd, vd, n = 4, 3, 9
    rng = np.random.default_rng(11)
    q, k, v = rng.uniform(-1, 1, (n, kd)), rng.uniform(-1, 1, (n, kd)), rng.uniform(-1, 1, (n, vd))
    g, beta = -rng.uniform(0, 1, n), rng.uniform(0, 1, n)

    def run(a, c, state, init):
        return gdn_f64(q[a:a + c], k[a:a + c], v[a:a + c], g[a:a + c], beta[a:a + c], state, [0], [0, c], kh=1, vh=1,
                       kd=kd, vd=vd, scale=0.5, init=init, l2=True, tokens=c, batch=1).ravel()

    whole = np.zeros(kd * vd, np.float32)
    full = run(0, n, whole, False)
    split = np.zeros(kd * vd, np.float32)
    two = np.concatenate([run(0, 4, split, False), run(4, 5, split, True)])
    assert np.max(np.abs(full - two)) < 1e-6 and np.max(np.abs(whole - split)) < 1e-6
    steps = np.zeros(kd * vd, np.float32)
    dec = np.concatenate([run(t, 1, steps, t > 0) for t in range(n)])
    assert np.max(np.abs(full - dec)) < 1e-5


@pytest.mark.parametrize("init", [True, False])
def test_gdn_shared_slots_run_in_batch_order(init):
    """Sequences of one call that share a slot run in batch order (CpuOps.Hybrid.cs:67-149 is one sequential loop):
    the multi-threaded call equals one single-sequence call per sequence, made one after another on the same pool."""
    rng = np.random.default_rng(17)
    lens, slots = [5, 7, 1, 0, 3], [2, 2, 4, 2, 2]
    d = cases.make_gdn(rng, lens, 6, slots=slots)
    out, pool = cases.oracle_gdn(d, use_initial_state=init, threads=8)
    seq_pool = d.pool.copy()
    seq_out = np.zeros_like(out)
    for b, n in enumerate(lens):
        t0 = int(d.cu[b])
        one = cases.GdnData(d.fused[t0:t0 + n].copy(), d.g[t0:t0 + n].copy(), d.beta[t0:t0 + n].copy(), seq_pool,
                            np.array([slots[b]], np.int32), np.array([0, n], np.int32), [n])
        o, seq_pool = cases.oracle_gdn(one, use_initial_state=init, threads=1)
        seq_out[t0:t0 + n] = o
    assert np.array_equal(out, seq_out) and np.array_equal(pool, seq_pool)


def test_gdn_scale_zero_means_inverse_root_kdim():
    def run(scale):
        return gdn_f64([1, 2, 3, 4], [0.5] * 4, [1], [0], [1], np.zeros(4, np.float32), [0], [0, 1], kh=1, vh=1, kd=4,
                       vd=1, scale=scale, init=False, l2=False, tokens=1, batch=1)[0, 0, 0]

    assert abs(run(0.5) - run(0.0)) < 1e-14


def test_gdn_strided_views_equal_contiguous_copies():
    rng = np.random.default_rng(3)
    d = cases.make_gdn(rng, [7, 5], 4, slots=[2, 0])
    out_s, pool_s = cases.oracle_gdn(d, threads=1)
    # Contiguous copies of the three column slices through the same function.
    out_c = np.zeros_like(out_s)
    pool_c = d.pool.copy()
    oracle.gated_delta_rule(d.view(0), d.view(1), d.view(2), d.g, d.beta, out_c, pool_c, d.slots, d.cu, batch=2,
                            tokens=12, k_heads=16, v_heads=16, k_dim=128, v_dim=128, bf16=True, beta_bf16=True)
    assert np.array_equal(out_s, out_c) and np.array_equal(pool_s, pool_c)


def test_gdn_strided_call_reads_only_the_view():
    """q_stride/k_stride/v_stride views of the fused buffer: the oracle given the fused buffer itself with strides
    6144 and column offsets equals the contiguous call."""
    rng = np.random.default_rng(8)
    d = cases.make_gdn(rng, [6, 2], 3, slots=[1, 2])
    out_c, pool_c = cases.oracle_gdn(d, threads=1)
    out_s = np.zeros_like(out_c)
    pool_s = d.pool.copy()
    fused = d.fused
    oracle.gated_delta_rule(fused, np.ascontiguousarray(fused[:, cases.ROW:]), np.ascontiguousarray(fused[:, 2 * cases.ROW:]),
                            d.g, d.beta, out_s, pool_s, d.slots, d.cu, batch=2, tokens=8, k_heads=16, v_heads=16,
                            k_dim=128, v_dim=128, q_stride=cases.FUSED, k_stride=cases.FUSED - cases.ROW,
                            v_stride=cases.FUSED - 2 * cases.ROW, bf16=True, beta_bf16=True)
    assert np.array_equal(out_s, out_c) and np.array_equal(pool_s, pool_c)


# ---- plan region -------------------------------------------------------------------------------------------------------

def test_plan_region_slot_mapping_closed_form():
    seqs = [dict(token_start=0, token_count=3, position_offset=0, kv_length=3, blocks=[7]),
            dict(token_start=3, token_count=1, position_offset=20, kv_length=21, blocks=[2, 9]),
            dict(token_start=4, token_count=18, position_offset=14, kv_length=32, blocks=[4, 1])]
    q_indptr, cu, kv_indptr, kv_indices, last, slots = oracle.plan_region(seqs, 16)
    assert list(q_indptr) == [0, 3, 4, 22] and list(cu) == [0, 3, 4, 22]
    assert list(kv_indptr) == [0, 1, 3, 5] and list(kv_indices) == [7, 2, 9, 4, 1]
    assert list(last) == [3, 5, 16]
    want = [7 * 16 + 0, 7 * 16 + 1, 7 * 16 + 2, 9 * 16 + 4] + [(4 if p < 16 else 1) * 16 + p % 16 for p in range(14, 32)]
    assert list(slots) == want



def test_plan_region_reference_hand_case():
    """PlanAndResultTests.cs:25-45: a 3-token prefill on block 5 and a 1-token decode at position 17 on blocks [2, 7]."""
    seqs = [dict(token_start=0, token_count=3, position_offset=0, kv_length=3, blocks=[5]),
            dict(token_start=3, token_count=1, position_offset=17, kv_length=18, blocks=[2, 7])]
    q_indptr, cu, kv_indptr, kv_indices, last, slots = oracle.plan_region(seqs, 16)
    assert list(slots) == [80, 81, 82, 7 * 16 + 1]
    assert list(q_indptr) == [0, 3, 4] and list(cu) == [0, 3, 4]
    assert list(kv_indptr) == [0, 1, 3] and list(kv_indices) == [5, 2, 7] and list(last) == [3, 2]

# ---- Gated DeltaNet layer neighbours --------------------------------------------------------------------------------
# Pinned by the reference's hand cases (tests/Starlings.Roost.Ops.Tests/GatingOpsTests.cs, HybridTests.cs:249-385) and by
# transformers 5.20.1's own float32 tensors, which the reference's tests hold as a fixture
# (Reference/qwen35-gating-cases.json, copied as data to tests/golden/qwen35_gating_cases.json).

import json
from pathlib import Path

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "qwen35_gating_cases.json").read_text())
LN2, LN3 = math.log(2), math.log(3)


def _f64(*v):
    return np.array(v, dtype=np.float64)


def _fx(case, key, dtype=np.float32):
    return np.array(GOLDEN[case][key], dtype=dtype)


def _rel(got, want, rel):
    """GatingReferenceTests.Rel: |got - want| <= rel * max(|want|, 1e-6) elementwise."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert (np.abs(got - want) <= rel * np.maximum(np.abs(want), 1e-6)).all()


def test_golden_fixture_is_the_pinned_reference():
    assert GOLDEN["transformers"] == "5.20.1"
    assert GOLDEN["modeling_qwen3_5_sha256"].startswith("b48635f7")


def test_gates_hand_case():
    """GatingOpsTests.GatesHandComputed: x = a + dt_bias = 0, 25, -1, 20 (softplus returns x above 20 only)."""
    a, b = _f64(1, 24, 0, 19), _f64(0, LN3, -LN3, 0)
    g, beta = np.zeros(4), np.zeros(4)
    oracle.gdn_gates(a, b, _f64(0, LN2), _f64(-1, 1), g, beta, tokens=2, v_heads=2)
    np.testing.assert_allclose(g, [-LN2, -50.0, -math.log(1 + math.exp(-1)), -2 * math.log(1 + math.exp(20))],
                               rtol=0, atol=1e-14)
    np.testing.assert_allclose(beta, [0.5, 0.75, 0.25, 0.5], rtol=0, atol=1e-15)


def test_gates_strided_views_and_output_types():
    """GatingOpsTests.GatesReadStridedViewsAndWriteEachSpansType: a at column 0 and b at column 2 of [tokens, 5] rows;
    g float32, beta bf16, a_log float32."""
    fused = _f64(0, 0, 0, 0, 99, 0, 0, 0, 0, 99)
    g, beta = np.zeros(4, np.float32), np.zeros(4, np.uint16)
    oracle.gdn_gates(fused, np.ascontiguousarray(fused[2:]), np.array([0, LN2], np.float32), _f64(0, 0), g, beta,
                     tokens=2, v_heads=2, a_stride=5, b_stride=5)
    np.testing.assert_allclose(g, [-LN2, -2 * LN2, -LN2, -2 * LN2], rtol=1e-6)
    assert list(oracle.bf16_to_f64(beta)) == [0.5] * 4
    with pytest.raises(oracle.OracleError):
        oracle.gdn_gates(fused, fused, _f64(0, 0), _f64(0, 0), np.zeros(4), np.zeros(4), tokens=2, v_heads=2,
                         a_stride=1)


def test_gates_match_transformers():
    c = GOLDEN["linear"]
    t, vh = c["tokens"], c["v_heads"]
    g, beta = np.zeros(t * vh), np.zeros(t * vh)
    oracle.gdn_gates(_fx("linear", "a"), _fx("linear", "b"), _fx("linear", "a_log"), _fx("linear", "dt_bias"), g, beta,
                     tokens=t, v_heads=vh)
    _rel(g, _fx("linear", "g"), 4e-7)
    _rel(beta, _fx("linear", "beta"), 4e-7)
    x = _fx("linear", "a", np.float64).reshape(t, vh)[:, 0] + c["dt_bias"][0]
    assert (x > 20).any() and (x < -20).any() and ((x > 0) & (x < 20)).any()  # both sides of the threshold


def test_gated_rms_norm_hand_cases():
    """GatingOpsTests: rows [3, 4] and [-1, 2], eps 0, weight [1, 0.5] as stored; in place with eps 1; a float32
    weight under bf16 activations."""
    o = np.zeros(4)
    oracle.gated_rms_norm(_f64(3, 4, -1, 2), _f64(0, LN3, LN3, LN3), _f64(1, 0.5), o, rows=2, dim=2, eps=0.0)
    s3 = LN3 * 0.75
    np.testing.assert_allclose(o, [0, 4 / math.sqrt(12.5) * 0.5 * s3, -1 / math.sqrt(2.5) * s3,
                                   2 / math.sqrt(2.5) * 0.5 * s3], rtol=0, atol=1e-15)
    x = _f64(1, 1)
    oracle.gated_rms_norm(x, _f64(10, 10), _f64(2, 2), x, rows=1, dim=2, eps=1.0)
    np.testing.assert_allclose(x, [2 / math.sqrt(2) * 10 / (1 + math.exp(-10))] * 2, rtol=0, atol=1e-14)
    xb, gb = oracle.to_bf16([1, 1]), oracle.to_bf16([16, 16])
    ob = np.zeros(2, np.uint16)
    oracle.gated_rms_norm(xb, gb, np.array([1.5, 0.25], np.float32), ob, rows=1, dim=2, eps=0.0)
    assert list(oracle.bf16_to_f64(ob)) == [24.0, 4.0]


def test_gated_rms_norm_matches_transformers_and_discriminates():
    c = GOLDEN["linear"]
    rows, dim = c["tokens"] * c["v_heads"], c["v_dim"]
    core, z, w = _fx("linear", "core"), _fx("linear", "z"), _fx("linear", "norm_weight")
    o = np.zeros(rows * dim, np.float32)
    oracle.gated_rms_norm(core, z, w, o, rows=rows, dim=dim, eps=c["eps"])
    want = _fx("linear", "norm_out")
    _rel(o, want, 4e-7)
    wrong = np.zeros_like(o)  # a zero-centred weight (1 + w) is far off
    oracle.gated_rms_norm(core, z, (1 + w).astype(np.float32), wrong, rows=rows, dim=dim, eps=c["eps"])
    assert np.abs(wrong - want).max() > 0.1


def test_sigmoid_mul_hand_case_in_place_and_transformers():
    o = np.zeros(4)
    x, gate = _f64(2, -4, 6, 1), _f64(0, LN3, -LN3, -800)
    oracle.sigmoid_mul(x, gate, o)
    np.testing.assert_allclose(o, [1, -3, 1.5, 0], rtol=0, atol=1e-15)
    oracle.sigmoid_mul(x, gate, x)
    np.testing.assert_allclose(x, [1, -3, 1.5, 0], rtol=0, atol=1e-15)
    attn, gate = _fx("attention", "attn"), _fx("attention", "gate")
    o = np.zeros_like(attn)
    oracle.sigmoid_mul(attn, gate, o)
    _rel(o, _fx("attention", "gated"), 4e-7)


def test_gdn_oracle_matches_transformers_delta_rule():
    """GatingReferenceTests.GatedDeltaRuleNormalisesQAndKInsideTheOp: transformers' q, k, v (before its l2 norm), g and
    beta from a zero state give its core output; without the in-op norm the result is far off."""
    c = GOLDEN["linear"]
    t, kh, vh, kd, vd = c["tokens"], c["k_heads"], c["v_heads"], c["k_dim"], c["v_dim"]
    core = _fx("linear", "core", np.float64)
    tol = 1e-5 * np.abs(core).max()

    def run(l2):
        out = np.zeros(t * vh * vd, np.float32)
        state = np.zeros(vh * kd * vd, np.float32)
        oracle.gated_delta_rule(_fx("linear", "q"), _fx("linear", "k"), _fx("linear", "v"), _fx("linear", "g"),
                                _fx("linear", "beta"), out, state, np.zeros(1, np.int32), np.array([0, t], np.int32),
                                batch=1, tokens=t, k_heads=kh, v_heads=vh, k_dim=kd, v_dim=vd, use_initial_state=False,
                                l2_norm_qk=l2)
        return out.astype(np.float64)

    assert np.abs(run(True) - core).max() <= tol
    assert np.abs(run(False) - core).max() > 100 * tol


def _conv(x, w, bias, state, slots, cu, *, batch, tokens, ch, width, silu):
    y = np.zeros(tokens * ch)
    oracle.causal_conv1d(x, w, bias, y, state, np.array(slots, np.int32), np.array(cu, np.int32), batch=batch,
                         tokens=tokens, channels=ch, width=width, silu=silu)
    return y


def test_causal_conv1d_hand_cases():
    """HybridTests.cs:249-277: width 3, state [1, 2], weights [1, 10, 100]; a one-token sequence with bias and silu."""
    st = _f64(1, 2)
    y = _conv(_f64(3, 4), _f64(1, 10, 100), None, st, [0], [0, 2], batch=1, tokens=2, ch=1, width=3, silu=False)
    assert list(y) == [321.0, 432.0] and list(st) == [3.0, 4.0]
    st = _f64(1, 2)
    y = _conv(_f64(3), _f64(1, 10, 100), _f64(-5), st, [0], [0, 1], batch=1, tokens=1, ch=1, width=3, silu=True)
    pre = 1 + 20 + 300 - 5
    assert abs(y[0] - pre / (1 + math.exp(-pre))) < 1e-10 and list(st) == [2.0, 3.0]


def test_causal_conv1d_one_call_equals_token_calls_and_independent_convolution():
    """HybridTests.cs:280-359: one call = token-by-token calls, other slots untouched, final state = the last
    width - 1 inputs; two packed sequences from zero states against a direct convolution in numpy."""
    rng = np.random.default_rng(3)
    ch, width, n = 3, 4, 7
    xs, ws = rng.uniform(-1, 1, n * ch), rng.uniform(-1, 1, ch * width)
    init = rng.uniform(-1, 1, 2 * ch * (width - 1))
    st = init.copy()
    y = _conv(xs, ws, None, st, [1], [0, n], batch=1, tokens=n, ch=ch, width=width, silu=True)
    st2 = init.copy()
    steps = [_conv(xs[t * ch:(t + 1) * ch].copy(), ws, None, st2, [1], [0, 1], batch=1, tokens=1, ch=ch, width=width,
                   silu=True) for t in range(n)]
    assert np.array_equal(y, np.concatenate(steps)) and np.array_equal(st, st2)
    assert np.array_equal(st[:ch * (width - 1)], init[:ch * (width - 1)])
    last = xs.reshape(n, ch)[n - (width - 1):].T  # [ch, width - 1], oldest first
    assert np.array_equal(st[ch * (width - 1):].reshape(ch, width - 1), last)
    # Two packed sequences from zero states.
    ch, width, lens = 2, 3, [4, 2]
    xs, ws = rng.uniform(-1, 1, 6 * ch), rng.uniform(-1, 1, ch * width)
    y = _conv(xs, ws, None, np.zeros(2 * ch * (width - 1)), [0, 1], [0, 4, 6], batch=2, tokens=6, ch=ch, width=width,
              silu=False)
    x2, w2 = xs.reshape(6, ch), ws.reshape(ch, width)
    start = 0
    for ln in lens:
        for t in range(ln):
            for c in range(ch):
                want = sum(w2[c, j] * x2[start + t - (width - 1) + j, c] for j in range(width)
                           if t - (width - 1) + j >= 0)
                assert abs(y[(start + t) * ch + c] - want) < 1e-13
        start += ln


def test_state_copy_and_snapshot_are_ordered_byte_copies():
    """HybridTests.cs:362-385: slot 2 <- slot 0, then slot 0 <- slot 1 (NaN and -0 kept bit for bit); snapshot and
    restore; a slot outside the pool is refused."""
    pool = np.array([1.5, -0.0, np.nan, 4, 5, 6], np.float32)
    oracle.state_copy(pool, np.array([0, 2, 1, 0], np.int32), slot_bytes=8)
    bits = pool.view(np.uint32)
    assert bits[0] == np.array([np.nan], np.float32).view(np.uint32)[0] and pool[1] == 4
    assert pool[4] == 1.5 and bits[5] == 0x80000000
    snaps = np.zeros(4, np.float32)
    oracle.state_snapshot(pool, snaps, np.array([2, 1], np.int32), slot_bytes=8, restore=False)
    assert list(snaps.view(np.uint32)) == [0, 0, np.float32(1.5).view(np.uint32), 0x80000000]
    pool2 = np.zeros(6, np.float32)
    oracle.state_snapshot(pool2, snaps, np.array([2, 1], np.int32), slot_bytes=8, restore=True)
    assert list(pool2.view(np.uint32)) == [0, 0, 0, 0, np.float32(1.5).view(np.uint32), 0x80000000]
    with pytest.raises(oracle.OracleError):
        oracle.state_copy(pool, np.array([3, 0], np.int32), slot_bytes=8)


# ---- QkNorm, Rope and the fused QkvQkNormRopeCacheWrite (CpuOps.cs:63-175, CpuOps.Fused.cs:37-95) ----

ROPE_GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "rope_llama3_cases.json").read_text())


def test_qk_norm_hand_case_and_strides():
    """BasicOpsTests.cs:35-46: one token, q heads [3, 4] and [6, 8] with weight 1, k head [0, 5] with weight [2, 3]."""
    q, k = np.array([3.0, 4, 6, 8]), np.array([0.0, 5])
    oracle.qk_norm(q, k, np.ones(2), np.array([2.0, 3]), tokens=1, q_heads=2, kv_heads=1, head_dim=2, eps=0.0)
    r, r2 = 1 / math.sqrt(12.5), 1 / math.sqrt(50)
    np.testing.assert_allclose(q, [3 * r, 4 * r, 6 * r2, 8 * r2], rtol=1e-15)
    np.testing.assert_allclose(k, [0.0, 5 / math.sqrt(12.5) * 3], rtol=1e-15)
    # Rows at a token stride (q heads inside a wider row) give what the contiguous rows give; padding is untouched.
    rng = np.random.default_rng(3)
    t, hq, hk, hd = 3, 2, 1, 8
    qs, ks = rng.standard_normal(t * 24), rng.standard_normal(t * 12)
    qc = qs.reshape(t, 24)[:, :hq * hd].copy().reshape(-1)
    kc = ks.reshape(t, 12)[:, :hk * hd].copy().reshape(-1)
    qw, kw = rng.standard_normal(hd), rng.standard_normal(hd)
    pad_q, pad_k = qs.reshape(t, 24)[:, hq * hd:].copy(), ks.reshape(t, 12)[:, hk * hd:].copy()
    oracle.qk_norm(qs, ks, qw, kw, tokens=t, q_heads=hq, kv_heads=hk, head_dim=hd, eps=1e-6, q_stride=24, k_stride=12)
    oracle.qk_norm(qc, kc, qw, kw, tokens=t, q_heads=hq, kv_heads=hk, head_dim=hd, eps=1e-6)
    assert np.array_equal(qs.reshape(t, 24)[:, :hq * hd].reshape(-1), qc)
    assert np.array_equal(ks.reshape(t, 12)[:, :hk * hd].reshape(-1), kc)
    assert np.array_equal(qs.reshape(t, 24)[:, hq * hd:], pad_q) and np.array_equal(ks.reshape(t, 12)[:, hk * hd:], pad_k)
    # With unit weights and eps 0 every normalised head has mean square 1.
    x = rng.standard_normal(5 * 16)
    oracle.qk_norm(x, np.zeros(5 * 16), np.ones(16), np.ones(16), tokens=5, q_heads=1, kv_heads=1, head_dim=16,
                   eps=0.0)
    np.testing.assert_allclose((x.reshape(5, 16) ** 2).mean(axis=1), 1.0, rtol=1e-14)


def _rope1(x, pos, hd, rot=0, interleaved=False, theta=100.0, llama3=None):
    q, k = np.array(x, np.float64), np.array(x, np.float64)
    oracle.rope(q, k, np.array([pos], np.int32), tokens=1, q_heads=1, kv_heads=1, head_dim=hd, rotary_dim=rot,
                interleaved=interleaved, theta=theta, llama3=llama3)
    assert np.array_equal(q, k)
    return q


def test_rope_hand_cases():
    """BasicOpsTests.cs:65-116."""
    a0, a1 = 2.0, 0.2  # head dim 4, theta 100: frequencies 1 and 0.1; position 2
    np.testing.assert_allclose(_rope1([1, 2, 3, 4], 2, 4),
                               [math.cos(a0) - 3 * math.sin(a0), 2 * math.cos(a1) - 4 * math.sin(a1),
                                3 * math.cos(a0) + math.sin(a0), 4 * math.cos(a1) + 2 * math.sin(a1)], rtol=1e-14)
    np.testing.assert_allclose(_rope1([1, 2, 3, 4], 2, 4, interleaved=True),
                               [math.cos(a0) - 2 * math.sin(a0), 2 * math.cos(a0) + math.sin(a0),
                                3 * math.cos(a1) - 4 * math.sin(a1), 4 * math.cos(a1) + 3 * math.sin(a1)], rtol=1e-14)
    y = _rope1([1, 2, 3, 4], 1, 4, rot=2)
    assert y[2] == 3.0 and y[3] == 4.0 and abs(y[0] - (math.cos(1.0) - 2 * math.sin(1.0))) < 1e-14
    assert list(_rope1([1, 2, 3, 4], 0, 4)) == [1.0, 2.0, 3.0, 4.0]
    # Llama 3: head dim 8, theta 1e6, original 8192, low 1, high 4, factor 8.
    y = _rope1([1, 1, 1, 1, 0, 0, 0, 0], 1000, 8, theta=1e6, llama3=(8.0, 1.0, 4.0, 8192))
    f = [float(np.float32(1e6)) ** (-2.0 * i / 8) for i in range(4)]
    smooth = (8192.0 / (2 * math.pi / f[2]) - 1) / (4 - 1)
    scaled = [f[0], f[1], (1 - smooth) * f[2] / 8 + smooth * f[2], f[3] / 8]
    for i in range(4):
        assert abs(math.cos(1000 * scaled[i]) - y[i]) < 1e-11 and abs(math.sin(1000 * scaled[i]) - y[i + 4]) < 1e-11
    with pytest.raises(oracle.OracleError):
        _rope1([1, 2, 3, 4], 1, 4, rot=3)


@pytest.mark.parametrize("case", ROPE_GOLDEN["cases"], ids=lambda c: c["name"])
def test_rope_llama3_matches_transformers(case):
    """RopeScalingTests.cs:105-127: a head of ones then zeros comes out as [cos, sin] of its position's angles, against
    transformers' own rows."""
    hd, pos, p = case["head_dim"], np.array(case["positions"], np.int32), case["params"]
    q = np.array([1.0 if i % hd < hd // 2 else 0.0 for i in range(len(pos) * hd)])
    k = np.zeros(len(pos) * hd)
    oracle.rope(q, k, pos, tokens=len(pos), q_heads=1, kv_heads=1, head_dim=hd, theta=case["theta"],
                llama3=(p["factor"], p["low_freq_factor"], p["high_freq_factor"], p["original_max_position_embeddings"]))
    np.testing.assert_allclose(q, case["cos_sin_rows"], rtol=0, atol=1e-9)


def test_rope_rotation_laws():
    """Each pair keeps its norm, and rotating by p1 then by p2 equals rotating by p1 + p2 (NeoX and interleaved,
    partial width)."""
    rng = np.random.default_rng(11)
    hd, rot = 16, 12
    for inter in (False, True):
        x = rng.standard_normal(hd)
        a = _rope1(x, 37, hd, rot=rot, interleaved=inter, theta=1e4)
        b = _rope1(_rope1(x, 30, hd, rot=rot, interleaved=inter, theta=1e4), 7, hd, rot=rot, interleaved=inter,
                   theta=1e4)
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-13)
        pairs = [(2 * i, 2 * i + 1) for i in range(rot // 2)] if inter else [(i, i + rot // 2) for i in range(rot // 2)]
        for i, j in pairs:
            assert abs(math.hypot(a[i], a[j]) - math.hypot(x[i], x[j])) < 1e-13
        assert np.array_equal(a[rot:], x[rot:])


def test_fused_qkv_is_its_parts_and_leaves_qkv_alone():
    """FusedOpsTests.cs:48-97 on the oracle: the fused call equals QkNorm, Rope and CacheWrite called in order, a -1 slot
    writes nothing, the qkv rows are left as they were; bf16 rows widen exactly into an f32 pool."""
    rng = np.random.default_rng(9)
    tokens, hq, hk, hd, bs, blocks = 5, 4, 2, 8, 4, 4
    qw, kw = hq * hd, hk * hd
    row = qw + 2 * kw
    qkv = cases.bf16_bits(rng.uniform(-1, 1, tokens * row).astype(np.float32))
    qn, kn = (cases.bf16_bits(rng.uniform(0.9, 1.1, hd).astype(np.float32)) for _ in range(2))
    pos = np.array([7, 8, 9, 0, 1], np.int32)
    slots = np.array([3, 12, -1, 5, 6], np.int64)
    before = qkv.copy()
    q_out = np.zeros(tokens * qw, np.uint16)
    kc, vc = np.zeros(blocks * bs * kw, np.uint16), np.zeros(blocks * bs * kw, np.uint16)
    oracle.qkv_qk_norm_rope_cache_write(qkv, q_out, qn, kn, pos, kc, vc, slots, tokens=tokens, q_heads=hq,
                                        kv_heads=hk, head_dim=hd, page_size=bs, eps=1e-6, theta=1e6)
    assert np.array_equal(qkv, before)
    rows = qkv.reshape(tokens, row)
    q = rows[:, :qw].copy().reshape(-1)
    k = rows[:, qw:qw + kw].copy().reshape(-1)
    v = rows[:, qw + kw:].copy().reshape(-1)
    oracle.qk_norm(q, k, qn, kn, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, eps=1e-6)
    oracle.rope(q, k, pos, tokens=tokens, q_heads=hq, kv_heads=hk, head_dim=hd, theta=1e6)
    assert np.array_equal(q_out, q)
    kr, vr = kc.reshape(-1, kw), vc.reshape(-1, kw)
    for t, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(kr[s], k.reshape(tokens, kw)[t]) and np.array_equal(vr[s], v.reshape(tokens, kw)[t])
    written = {int(s) for s in slots if s >= 0}
    assert all(not kr[r].any() and not vr[r].any() for r in range(blocks * bs) if r not in written)
    kc32, vc32 = np.zeros(blocks * bs * kw, np.float32), np.zeros(blocks * bs * kw, np.float32)
    oracle.qkv_qk_norm_rope_cache_write(qkv, q_out, qn, kn, pos, kc32, vc32, slots, tokens=tokens, q_heads=hq,
                                        kv_heads=hk, head_dim=hd, page_size=bs, eps=1e-6, theta=1e6)
    assert np.array_equal(kc32.view(np.uint32) >> 16, kc.astype(np.uint32))
    assert np.array_equal(vc32.view(np.uint32) >> 16, vc.astype(np.uint32))
