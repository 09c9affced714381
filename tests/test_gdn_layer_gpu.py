"""The Gated DeltaNet layer's neighbour ops on the GPU through the C ABI against the CpuOps oracle: GatedDeltaRuleGates,
GatedRmsNorm, SigmoidMul, CausalConv1d, RecurrentStateCopy and RecurrentStateSnapshot.

Tolerances: an output the library rounds to bf16 from fp32 and the oracle from double may differ by one rounding step,
so bf16 outputs must lie within one bf16 ulp of the oracle's (an ulp is 2^-8 to 2^-7 of the value, so |d| <= 2^-7 |ref|,
far inside BASELINE's 2e-2 / 1e-2 bar);
fp32 outputs within 2e-5 relative (the fp32 exp and log are accurate to a few ulps). Conv states and the state copies
are bit-exact (they move input bits)."""
import zlib

import numpy as np
import pytest

import cases
import oracle
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev, to_dev

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7  # one bf16 ulp is at most this fraction of the value


def assert_bf16_within_ulp(got_bits, want_bits, what):
    got, want = oracle.bf16_to_f64(got_bits), oracle.bf16_to_f64(want_bits)
    assert np.all(np.isfinite(got)), what
    bad = np.abs(got - want) > BF16_ULP * np.abs(want) + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} elements beyond one bf16 ulp, e.g. got {got[bad][:4]} want {want[bad][:4]}"


def assert_f32_rel(got, want, rel, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    scale = np.maximum(np.abs(want), 1e-6)
    r = np.abs(got - want) / scale
    i = int(np.argmax(r))
    assert (r <= rel).all(), f"{what}: max rel {r[i]:.3e} at element {i}: got {got[i]!r} want {want[i]!r}"


def test_gates_qwen35_layout(session):
    """a and b are columns of one [tokens, 64] projection row (b at 0, a at 16, stride 64), 16 value heads; a_log and
    dt_bias f32; g f32, beta bf16 -- how Qwen3.5 binds them. x = a + dt_bias spans both sides of softplus's threshold."""
    import torch

    rng = np.random.default_rng(61)
    tokens, vh, row = 300, 16, 64
    proj = rng.standard_normal((tokens, row)).astype(np.float32) * 8.0
    proj_bits = cases.bf16_bits(proj)
    a_log = (rng.standard_normal(vh) * 0.5).astype(np.float32)
    dt_bias = (rng.standard_normal(vh) * 10.0).astype(np.float32)
    a_view = np.ascontiguousarray(proj_bits[:, 16:16 + vh])
    b_view = np.ascontiguousarray(proj_bits[:, :vh])
    want_g, want_beta = np.zeros(tokens * vh, np.float32), np.zeros(tokens * vh, np.uint16)
    oracle.gdn_gates(a_view, b_view, a_log, dt_bias, want_g, want_beta, tokens=tokens, v_heads=vh)
    d_proj = to_dev(proj_bits, True)
    g = torch.full((tokens * vh,), float("nan"), dtype=torch.float32, device="cuda")
    beta = torch.zeros((tokens * vh,), dtype=torch.bfloat16, device="cuda")
    reach = (tokens - 1) * row + vh
    roost_amd.gated_delta_rule_gates(session, d_proj, d_proj, to_dev(a_log), to_dev(dt_bias), g, beta, tokens=tokens,
                                     v_heads=vh, a_stride=row, b_stride=row, a_len=reach, b_len=reach, a_offset=16,
                                     b_offset=0)
    assert_f32_rel(from_dev(g), want_g, 2e-5, "g")
    assert_bf16_within_ulp(from_dev(beta, True), want_beta, "beta")
    x = oracle.bf16_to_f64(a_view).reshape(tokens, vh) + dt_bias
    assert (x > 20).any() and (x < 20).any()


def test_gates_match_transformers_fixture(session):
    """transformers 5.20.1's own float32 inputs and outputs (the reference's fixture), all spans f32."""
    import torch

    c = __import__("test_oracle").GOLDEN["linear"]
    t, vh = c["tokens"], c["v_heads"]
    f = lambda k: np.array(c[k], np.float32)  # noqa: E731
    g = torch.zeros(t * vh, dtype=torch.float32, device="cuda")
    beta = torch.zeros(t * vh, dtype=torch.float32, device="cuda")
    roost_amd.gated_delta_rule_gates(session, to_dev(f("a")), to_dev(f("b")), to_dev(f("a_log")), to_dev(f("dt_bias")),
                                     g, beta, tokens=t, v_heads=vh)
    assert_f32_rel(from_dev(g), f("g"), 2e-5, "g vs transformers")
    assert_f32_rel(from_dev(beta), f("beta"), 2e-5, "beta vs transformers")


@pytest.mark.parametrize("rows,dim,bf16,in_place", [(300 * 16, 128, True, False), (77, 128, True, True),
                                                     (40, 7, False, False), (9, 1000, False, True),
                                                     (5, 4096, True, False), (33, 128, False, False),
                                                     (10, 16, True, True)])
def test_gated_rms_norm(session, rows, dim, bf16, in_place):
    import torch

    rng = np.random.default_rng(rows + dim)
    x = rng.standard_normal(rows * dim).astype(np.float32)
    z = (rng.standard_normal(rows * dim) * 2).astype(np.float32)
    w = (rng.standard_normal(dim) * 0.5 + 1).astype(np.float32)  # an f32 weight, as Qwen3.5 keeps it
    if bf16:
        x, z = cases.bf16_bits(x), cases.bf16_bits(z)
    want = np.zeros_like(x)
    oracle.gated_rms_norm(x, z, w, want, rows=rows, dim=dim, eps=1e-6)
    dx, dz = to_dev(x, bf16), to_dev(z, bf16)
    out = dx if in_place else torch.full_like(dx, float("nan"))
    roost_amd.gated_rms_norm(session, dx, dz, to_dev(w), out, rows=rows, dim=dim, eps=1e-6)
    got = from_dev(out, bf16)
    if bf16:
        assert_bf16_within_ulp(got, want, "gated rms norm")
    else:
        assert_f32_rel(got, want, 2e-5, "gated rms norm f32")


def test_gated_rms_norm_matches_transformers_fixture(session):
    import torch

    c = __import__("test_oracle").GOLDEN["linear"]
    rows, dim = c["tokens"] * c["v_heads"], c["v_dim"]
    f = lambda k: np.array(c[k], np.float32)  # noqa: E731
    out = torch.zeros(rows * dim, dtype=torch.float32, device="cuda")
    roost_amd.gated_rms_norm(session, to_dev(f("core")), to_dev(f("z")), to_dev(f("norm_weight")), out, rows=rows,
                             dim=dim, eps=c["eps"])
    want = f("norm_out")
    np.testing.assert_allclose(from_dev(out), want, rtol=2e-5, atol=2e-5 * np.abs(want).max())


@pytest.mark.parametrize("n,bf16,in_place", [(300 * 2048, True, False), (1001, True, True), (4096, False, False),
                                             (13, False, True)])
def test_sigmoid_mul(session, n, bf16, in_place):
    import torch

    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    gate = (rng.standard_normal(n) * 4).astype(np.float32)
    if bf16:
        x, gate = cases.bf16_bits(x), cases.bf16_bits(gate)
    want = np.zeros_like(x)
    oracle.sigmoid_mul(x, gate, want)
    dx = to_dev(x, bf16)
    out = dx if in_place else torch.full_like(dx, float("nan"))
    roost_amd.sigmoid_mul(session, dx, to_dev(gate, bf16), out, rows=1, dim=n)
    got = from_dev(out, bf16)
    if bf16:
        assert_bf16_within_ulp(got, want, "sigmoid mul")
    else:
        assert_f32_rel(got, want, 2e-5, "sigmoid mul f32")


def _conv_case(session, lens, slots, pool_slots, channels, width, silu, bias, bf16, state_f32, seed):
    import torch

    rng = np.random.default_rng(seed)
    tokens = int(sum(lens))
    x = rng.standard_normal(tokens * channels).astype(np.float32)
    w = (rng.standard_normal(channels * width) * 0.5).astype(np.float32)
    b = (rng.standard_normal(channels) * 0.1).astype(np.float32) if bias else None
    sl = width - 1
    st = rng.standard_normal(max(pool_slots * channels * sl, 1)).astype(np.float32)
    if bf16:
        x, w = cases.bf16_bits(x), cases.bf16_bits(w)
        b = cases.bf16_bits(b) if bias else None
    if not state_f32:
        st = cases.bf16_bits(st)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots = np.array(slots, np.int32)
    want = np.zeros_like(x)
    want_state = st.copy()
    # The oracle refuses out-of-pool slots; the library leaves them untouched and reads a zero history. Run the oracle
    # on the in-pool sequences only, with the others' rows computed from a zero history.
    ok = (slots >= 0) & (slots < pool_slots)
    for bi in range(len(lens)):
        if lens[bi] == 0:
            continue
        seg = slice(int(cu[bi]) * channels, int(cu[bi + 1]) * channels)
        y = np.zeros(lens[bi] * channels, x.dtype)
        if ok[bi]:
            oracle.causal_conv1d(np.ascontiguousarray(x[seg]), w, b, y, want_state, slots[bi:bi + 1],
                                 np.array([0, lens[bi]], np.int32), batch=1, tokens=lens[bi], channels=channels,
                                 width=width, silu=silu)
        else:
            zero = np.zeros(max(channels * sl, 1), want_state.dtype)
            oracle.causal_conv1d(np.ascontiguousarray(x[seg]), w, b, y, zero, np.zeros(1, np.int32),
                                 np.array([0, lens[bi]], np.int32), batch=1, tokens=lens[bi], channels=channels,
                                 width=width, silu=silu)
        want[seg] = y
    dx = to_dev(x, bf16)
    dst = to_dev(st, not state_f32)
    out = torch.full_like(dx, float("nan"))
    roost_amd.causal_conv1d(session, dx, to_dev(w, bf16), to_dev(b, bf16) if bias else None, out, dst, to_dev(slots),
                            to_dev(cu), batch=len(lens), tokens=tokens, channels=channels, width=width, silu=silu)
    return from_dev(out, bf16), want, from_dev(dst, not state_f32), want_state


@pytest.mark.parametrize("name,lens,slots,pool,channels,width,silu,bias,bf16,state_f32", [
    ("qwen35 mixed batch", [1, 5, 0, 300, 2, 1], [3, 0, 1, 5, 2, 4], 6, 6144, 4, True, False, True, False),
    ("out-of-pool slots read zeros", [4, 3], [-1, 7], 2, 6144, 4, True, False, True, False),
    ("f32 with bias, width 3, f32 state", [7, 1, 20], [1, 0, 2], 3, 40, 3, False, True, False, True),
    ("width 1 (no state)", [3, 4], [0, 1], 2, 24, 1, True, True, False, True),
    ("odd channels scalar path", [9, 2], [1, 0], 2, 13, 4, True, False, True, True),
    ("one sequence, ragged last tile", [45, 70], [1, 0], 2, 128, 4, True, True, True, False),
    # decode-shaped batches (fewer tokens than sequences x 32: the one-token-per-thread short form)
    ("decode 64 x 1, width 3, bias, f32 state", [1] * 64, list(range(63, -1, -1)), 64, 1024, 3, True, True, True, True),
    ("short rows, width 2, unslotted row", [2, 1, 3, 0, 1], [0, -1, 2, 3, 1], 4, 512, 2, False, True, True, False),
])
def test_causal_conv1d(session, name, lens, slots, pool, channels, width, silu, bias, bf16, state_f32):
    got, want, got_state, want_state = _conv_case(session, lens, slots, pool, channels, width, silu, bias, bf16,
                                                  state_f32, zlib.crc32(name.encode()) % 1000)
    if bf16:
        assert_bf16_within_ulp(got, want, f"{name} output")
    else:
        assert_f32_rel(got, want, 2e-5, f"{name} output")
    if width > 1:
        assert np.array_equal(got_state.view(np.uint8), want_state.view(np.uint8)), f"{name}: conv state not bit-exact"


def test_causal_conv1d_one_call_equals_token_calls(session):
    """HybridTests.cs:280-320 on the GPU: a 7-token call equals seven one-token calls chained through the slot."""
    import torch

    rng = np.random.default_rng(5)
    ch, width, n = 64, 4, 7
    x = cases.bf16_bits(rng.standard_normal(n * ch).astype(np.float32))
    w = cases.bf16_bits(rng.standard_normal(ch * width).astype(np.float32))
    init = cases.bf16_bits(rng.standard_normal(2 * ch * (width - 1)).astype(np.float32))
    slots = to_dev(np.array([1], np.int32))
    d_w = to_dev(w, True)
    st_a = to_dev(init, True)
    out_a = torch.zeros(n * ch, dtype=torch.bfloat16, device="cuda")
    roost_amd.causal_conv1d(session, to_dev(x, True), d_w, None, out_a, st_a, slots, to_dev(np.array([0, n], np.int32)),
                            batch=1, tokens=n, channels=ch, width=width, silu=True)
    st_b = to_dev(init, True)
    outs = []
    for t in range(n):
        o = torch.zeros(ch, dtype=torch.bfloat16, device="cuda")
        roost_amd.causal_conv1d(session, to_dev(np.ascontiguousarray(x[t * ch:(t + 1) * ch]), True), d_w, None, o, st_b,
                                slots, to_dev(np.array([0, 1], np.int32)), batch=1, tokens=1, channels=ch, width=width,
                                silu=True)
        outs.append(from_dev(o, True))
    assert np.array_equal(from_dev(out_a, True), np.concatenate(outs))
    assert np.array_equal(from_dev(st_a, True), from_dev(st_b, True))
    assert np.array_equal(from_dev(st_a, True)[:ch * (width - 1)], init[:ch * (width - 1)])  # slot 0 untouched


@pytest.mark.parametrize("slot_bytes,count", [(65536, 40), (4096, 600), (6, 40)])
def test_state_copy_long_chains_match_oracle(session, slot_bytes, count):
    """Many pairs over few slots: chains where a pair reads what an earlier one (adjacent or not) wrote and self
    copies, against the oracle's in-order byte copies; 600 pairs cross the kernel's 512-pair batch."""
    rng = np.random.default_rng(count + slot_bytes)
    slots = 6
    pool = rng.integers(0, 256, slots * slot_bytes, dtype=np.uint8)
    pairs = rng.integers(0, slots, 2 * count).astype(np.int32)
    want = pool.copy()
    oracle.state_copy(want, pairs, slot_bytes=slot_bytes)
    d = to_dev(pool)
    roost_amd.recurrent_state_copy(session, d, to_dev(pairs), slot_bytes=slot_bytes, count=count)
    assert np.array_equal(from_dev(d), want)


@pytest.mark.parametrize("slot_bytes", [8, 6, 65536])
def test_state_copy_and_snapshot_bit_exact(session, slot_bytes):
    """Ordered pair copies (a later pair sees an earlier pair's write), NaN and -0 bit patterns kept; 16-byte, word and
    byte paths."""
    rng = np.random.default_rng(slot_bytes)
    slots = 5
    pool = rng.integers(0, 256, slots * slot_bytes, dtype=np.uint8)
    pool[:4] = np.frombuffer(np.float32(np.nan).tobytes(), np.uint8)
    pairs = np.array([0, 2, 1, 0, 2, 4, 3, 3], np.int32)  # slot 4 gets slot 0's old bytes through slot 2
    want = pool.copy()
    oracle.state_copy(want, pairs, slot_bytes=slot_bytes)
    d = to_dev(pool)
    roost_amd.recurrent_state_copy(session, d, to_dev(pairs), slot_bytes=slot_bytes, count=4)
    assert np.array_equal(from_dev(d), want)
    snaps = np.zeros(3 * slot_bytes, np.uint8)
    sp = np.array([4, 1, 0, 2], np.int32)
    want_s = snaps.copy()
    oracle.state_snapshot(want, want_s, sp, slot_bytes=slot_bytes, restore=False)
    ds = to_dev(snaps)
    roost_amd.recurrent_state_snapshot(session, d, ds, to_dev(sp), slot_bytes=slot_bytes, count=2, restore=False)
    assert np.array_equal(from_dev(ds), want_s)
    fresh = np.zeros_like(pool)
    oracle.state_snapshot(fresh, want_s, sp, slot_bytes=slot_bytes, restore=True)
    dfresh = to_dev(np.zeros_like(pool))
    roost_amd.recurrent_state_snapshot(session, dfresh, ds, to_dev(sp), slot_bytes=slot_bytes, count=2, restore=True)
    assert np.array_equal(from_dev(dfresh), fresh)


def test_refusals(session):
    """Typed statuses before any launch (kernels/src/ops/gating.cu, causal_conv1d.cu, recurrent_state.cu)."""
    import torch

    x = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    run = lambda vid, p: session.run_raw(session.lib.entry(vid), p, None)  # noqa: E731
    p = roost_amd.sigmoid_mul_params(x, x, x[1:], rows=1, dim=32)
    assert run(roost_amd.SIGMOID_MUL_VARIANT, p) == abi.INVALID_ARGUMENT  # partial overlap
    p = roost_amd.gated_rms_norm_params(x, x, x, x, rows=2, dim=32, eps=-1.0)
    assert run(roost_amd.GATED_RMS_NORM_VARIANT, p) == abi.INVALID_ARGUMENT
    i8 = torch.zeros(64, dtype=torch.int32, device="cuda")
    p = roost_amd.sigmoid_mul_params(i8, i8, i8, rows=1, dim=32)
    assert run(roost_amd.SIGMOID_MUL_VARIANT, p) == abi.UNSUPPORTED
    g = torch.zeros(8, dtype=torch.float32, device="cuda")
    p = roost_amd.gated_delta_rule_gates_params(x, x, g, g, g, g, tokens=2, v_heads=4)
    assert run(roost_amd.GATES_VARIANT, p) == abi.INVALID_ARGUMENT  # g and beta overlap
    slots = torch.zeros(1, dtype=torch.int32, device="cuda")
    cu = torch.tensor([0, 2], dtype=torch.int32, device="cuda")
    st = torch.zeros(96, dtype=torch.bfloat16, device="cuda")
    p = roost_amd.causal_conv1d_params(x, x, None, x, st, slots, cu, batch=1, tokens=2, channels=32, width=17)
    assert run(roost_amd.CAUSAL_CONV1D_VARIANT, p) == abi.INVALID_ARGUMENT
    p = roost_amd.causal_conv1d_params(x, x, None, x, st, slots, cu, batch=1, tokens=2, channels=32, width=2)
    assert run(roost_amd.CAUSAL_CONV1D_VARIANT, p) == abi.INVALID_ARGUMENT  # input aliases output
    p = roost_amd.recurrent_state_copy_params(st, slots, slot_bytes=8, count=1)
    assert run(roost_amd.STATE_COPY_VARIANT, p) == abi.INVALID_ARGUMENT  # pairs too short for one pair
    torch.cuda.synchronize()
