"""GatedDeltaRule (chunk and recurrent variants) on the GPU through the C ABI vs the CpuOps oracle (reference harness:
kernels/tests/hybrid-conformance/GdnCases.cs:31-471). Tolerances: output max-abs 2e-2 and max-rel 1e-2; final state
max-rel 1e-3 (relative to |ref_i| + max|ref|), per BASELINE.json."""
import zlib

import numpy as np
import pytest

import cases
import oracle
import roost_amd
from cases import DIM, FUSED, HEADS, ROW
from roost_amd import abi
from test_attention_gpu import from_dev, to_dev

pytestmark = pytest.mark.gpu

VARIANTS = [roost_amd.RECURRENT_VARIANT, roost_amd.CHUNK_VARIANT]


class DevGdn:
    def __init__(self, d: cases.GdnData, strided=True):
        import torch

        self.d = d
        self.strided = strided
        self.fused = to_dev(d.fused, True)
        if not strided:
            self.q, self.k, self.v = (to_dev(d.view(i), True) for i in range(3))
        self.g = to_dev(d.g)
        self.beta = to_dev(d.beta, True)
        self.pool = to_dev(d.pool)
        self.slots = to_dev(d.slots)
        self.cu = to_dev(d.cu)
        self.out = torch.full((max(d.tokens, 1), HEADS, DIM), float("nan"), dtype=torch.bfloat16, device="cuda")

    def params(self, init=True, **over):
        d = self.d
        reach = 0 if d.tokens == 0 else (d.tokens - 1) * FUSED + ROW
        if self.strided:
            kw = dict(q_stride=FUSED, k_stride=FUSED, v_stride=FUSED, q_len=reach, k_len=reach, v_len=reach,
                      q_offset=0, k_offset=ROW, v_offset=2 * ROW)
            q = k = v = self.fused
        else:
            kw = {}
            q, k, v = self.q, self.k, self.v
        kw.update(batch=d.batch, tokens=d.tokens, use_initial_state=init, cu_seqlens_host=d.cu)
        kw.update(over)
        return roost_amd.gated_delta_rule_params(q, k, v, self.g, self.beta, self.out, self.pool, self.slots, self.cu,
                                                 **kw)


def run(session, dev: DevGdn, variant, init=True):
    p = dev.params(init)
    session.launch(session.lib.entry(variant), p, key=(dev.d.batch, dev.d.tokens))
    return from_dev(dev.out, True)[: dev.d.tokens], from_dev(dev.pool)


CASES = [
    ("packed [300,77,1500,64,1] init strided", [300, 77, 1500, 64, 1], True, True, 0.2, 11),
    ("packed [300,77,1500] no init strided", [300, 77, 1500], True, False, 0.2, 12),
    ("one 1000 contiguous init", [1000], False, True, 0.2, 13),
    ("chunk boundaries [64,128,65,1,0,63]", [64, 128, 65, 1, 0, 63], True, True, 0.2, 14),
    ("strong decay [200,40]", [200, 40], True, True, 2.5, 15),
    ("decode 4x1 strided init", [1, 1, 1, 1], True, True, 0.2, 21),
    ("packed [5,1,1] contiguous", [5, 1, 1], False, True, 0.2, 22),
    ("one of 3 no init", [3], True, False, 0.2, 23),
    ("decode with empty [1,0,1]", [1, 0, 1], True, True, 0.2, 24),
    ("32 x 1 serving decode", [1] * 32, True, True, 0.2, 26),
    # A mixed worker step: the recurrent variant hands sequences of 16 tokens or more to the chunk kernels.
    ("hybrid step [1,15,16,1,600,0,64,2]", [1, 15, 16, 1, 600, 0, 64, 2], True, True, 0.2, 27),
    ("hybrid step [17,1,1,1] no init", [17, 1, 1, 1], False, False, 0.2, 28),
]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("name,lens,strided,init,decay,seed", CASES, ids=[c[0] for c in CASES])
def test_matches_cpuops(session, variant, name, lens, strided, init, decay, seed):
    rng = np.random.default_rng(seed)
    pool_slots = 41
    d = cases.make_gdn(rng, lens, pool_slots, decay=decay)
    want_o, want_pool = cases.oracle_gdn(d, use_initial_state=init)
    dev = DevGdn(d, strided)
    got_o, got_pool = run(session, dev, variant, init)
    cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o), what="gdn output")
    owned = {int(d.slots[b]) for b in range(d.batch) if d.lens[b] > 0}
    for s in range(pool_slots):
        if s in owned:
            cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"state slot {s}")
        else:
            assert got_pool[s].tobytes() == d.pool[s].tobytes(), f"slot {s} was touched"


@pytest.mark.parametrize("variant", VARIANTS)
def test_negative_slot_runs_from_zero_and_is_not_written(session, variant):
    lens = [600, 70] if variant == roost_amd.CHUNK_VARIANT else [1, 1]  # 600 tokens: scanned in parts
    rng = np.random.default_rng(51)
    d = cases.make_gdn(rng, lens, 9, slots=[-1, 3])
    a = DevGdn(d)
    o_neg, pool_neg = run(session, a, variant, init=True)
    b = DevGdn(d)
    o_zero, _ = run(session, b, variant, init=False)
    n0 = lens[0]
    assert o_neg[:n0].tobytes() == o_zero[:n0].tobytes()
    for s in range(9):
        if s != 3:
            assert pool_neg[s].tobytes() == d.pool[s].tobytes()


@pytest.mark.parametrize("variant", VARIANTS)
def test_batch_invariance(session, variant):
    lens = [333, 200, 129] if variant == roost_amd.CHUNK_VARIANT else [1, 1, 1]
    rng = np.random.default_rng(31)
    many = cases.make_gdn(rng, lens, 9, slots=[4, 7, 2])
    n0 = lens[0]
    one = cases.GdnData(many.fused[:n0].copy(), many.g[:n0].copy(), many.beta[:n0].copy(), many.pool.copy(),
                        np.array([4], np.int32), np.array([0, n0], np.int32), [n0])
    o_many, p_many = run(session, DevGdn(many), variant)
    o_one, p_one = run(session, DevGdn(one), variant)
    assert o_many[:n0].tobytes() == o_one.tobytes()
    assert p_many[4].tobytes() == p_one[4].tobytes()


@pytest.mark.parametrize("variant", VARIANTS)
def test_deterministic(session, variant):
    rng = np.random.default_rng(77)
    # Distinct slots: sequences of one call that share a slot race (the routed path runs them side by side).
    d = cases.make_gdn(rng, [130, 7], 5, slots=[1, 3])
    o1, p1 = run(session, DevGdn(d), variant)
    o2, p2 = run(session, DevGdn(d), variant)
    assert o1.tobytes() == o2.tobytes() and p1.tobytes() == p2.tobytes()


SHARED_SLOT_CASES = [
    ("decode, three rows on slot 3", [1, 1, 1, 1, 1], [3, 1, 3, 3, 0], True),
    ("short rows, empty member, no init", [5, 7, 1, 0, 3], [2, 2, 4, 2, 2], False),
    ("routed call, short rows share a slot", [100, 5, 3, 1], [0, 1, 1, 2], True),
]


@pytest.mark.parametrize("name,lens,slots,init", SHARED_SLOT_CASES, ids=[c[0] for c in SHARED_SLOT_CASES])
def test_recurrent_shared_slots_run_in_batch_order(session, name, lens, slots, init):
    """Sequences of one recurrent call that share a state slot (and run on the recurrent kernel: shorter than 16
    tokens) run in batch order, as CpuOps runs them (CpuOps.Hybrid.cs:67-149): each starts from the state the one
    before it wrote, or from zero without use_initial_state. Against the oracle, and bit-identical on a second run
    (the variant registers DETERMINISTIC)."""
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    d = cases.make_gdn(rng, lens, 6, slots=slots)
    want_o, want_pool = cases.oracle_gdn(d, use_initial_state=init)
    o1, p1 = run(session, DevGdn(d), roost_amd.RECURRENT_VARIANT, init)
    o2, p2 = run(session, DevGdn(d), roost_amd.RECURRENT_VARIANT, init)
    assert o1.tobytes() == o2.tobytes() and p1.tobytes() == p2.tobytes()
    cases.assert_close(cases.bf16_values(o1), cases.bf16_values(want_o), what=f"{name} output")
    for s in set(slots):
        cases.assert_close(p1[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"{name} slot {s}")
    for s in set(range(6)) - set(slots):
        assert p1[s].tobytes() == d.pool[s].tobytes()


def test_config4_chunked_prefill_then_recurrent_decode(session):
    """4 x 4096 tokens, 16 heads x 128, beta = sigmoid(N(0,1)), g = -softplus(N(0,1)),
    S0 ~ N(0, 0.01); chunked prefill vs CpuOps; then recurrent decode steps on 128 states vs CpuOps."""
    rng = np.random.default_rng(4)
    d = cases.make_gdn(rng, [4096] * 4, 4, slots=[0, 1, 2, 3], baseline_style=True)
    want_o, want_pool = cases.oracle_gdn(d)
    got_o, got_pool = run(session, DevGdn(d), roost_amd.CHUNK_VARIANT)
    cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o), what="config 4 chunk output")
    for s in range(4):
        cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"config 4 state {s}")
    _recurrent_chain(session, rng, states=128, steps=128)


def _recurrent_chain(session, rng, states, steps):
    """`steps` recurrent decode calls of one token per sequence on `states` states, chained through the pool; every
    call's output is checked, and the final states after the last call. The CpuOps reference runs the whole chain as
    one call of `steps`-token sequences (one call over n tokens = n one-token calls: HybridTests.cs:174-220)."""
    dd = cases.make_gdn(rng, [1] * states, states, slots=list(range(states)), baseline_style=True)
    fused = np.empty((steps, states, FUSED), np.uint16)
    g = np.empty((steps, states, HEADS), np.float32)
    beta = np.empty((steps, states, HEADS), np.uint16)
    for t in range(steps):
        sd = cases.make_gdn(rng, [1] * states, states, slots=list(range(states)), baseline_style=True)
        fused[t], g[t], beta[t] = sd.fused, sd.g, sd.beta
    # Sequence-major copy for the one-call reference: sequence b's tokens are steps 0..steps-1 of state b.
    whole = cases.GdnData(np.ascontiguousarray(fused.transpose(1, 0, 2).reshape(-1, FUSED)),
                          np.ascontiguousarray(g.transpose(1, 0, 2).reshape(-1, HEADS)),
                          np.ascontiguousarray(beta.transpose(1, 0, 2).reshape(-1, HEADS)), dd.pool.copy(),
                          np.arange(states, dtype=np.int32),
                          (np.arange(states + 1) * steps).astype(np.int32), [steps] * states)
    want_o, want_pool = cases.oracle_gdn(whole)
    want_o = want_o.reshape(states, steps, HEADS, DIM)
    dev = DevGdn(dd)
    for t in range(steps):
        dev.fused.copy_(to_dev(fused[t], True))
        dev.g.copy_(to_dev(g[t]))
        dev.beta.copy_(to_dev(beta[t], True))
        p = dev.params()
        session.launch(session.lib.entry(roost_amd.RECURRENT_VARIANT), p, key=("chain", states))
        if t % 16 == 0 or t == steps - 1:
            got_o = from_dev(dev.out, True)[:states]
            cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o[:, t]), what=f"decode step {t}")
    got_pool = from_dev(dev.pool)
    for s in range(states):
        cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL,
                           what=f"state {s} after {steps} steps")


def test_rejections(session):
    rng = np.random.default_rng(41)
    d = cases.make_gdn(rng, [2, 3], 4, slots=[1, 3])
    dev = DevGdn(d)
    rec = session.lib.entry(roost_amd.RECURRENT_VARIANT)
    chunk = session.lib.entry(roost_amd.CHUNK_VARIANT)

    def status(entry, p, ws=None):
        return session.run_raw(entry, p, ws)

    p = dev.params(q_stride=ROW - 8)
    assert status(rec, p) == abi.INVALID_ARGUMENT
    p = dev.params()
    p.v.length -= 1
    assert status(rec, p) == abi.INVALID_ARGUMENT
    # Value heads must be 1 to 8 whole groups of the key heads.
    assert status(rec, dev.params(k_heads=3, v_heads=16)) == abi.UNSUPPORTED
    assert status(rec, dev.params(k_heads=1, v_heads=16)) == abi.UNSUPPORTED
    assert status(rec, dev.params(k_dim=64, v_dim=64)) == abi.UNSUPPORTED
    assert status(rec, dev.params(l2_norm_qk=False)) == abi.UNSUPPORTED
    p = dev.params()
    p.beta.dtype = abi.DTYPE_F32
    assert status(rec, p) == abi.UNSUPPORTED
    p = dev.params()
    p.g.address += 4
    assert status(rec, p) == abi.INVALID_ARGUMENT
    p = dev.params()
    p.struct_size = 64
    assert status(rec, p) == abi.ABI_MISMATCH
    p = dev.params()
    p.state.length = HEADS * DIM * DIM + 5
    assert status(rec, p) == abi.INVALID_ARGUMENT
    # A call that may hold a sequence of 16 tokens or more needs the recurrent variant's workspace.
    long_dev = DevGdn(cases.make_gdn(rng, [20, 1], 4, slots=[0, 2]))
    assert status(rec, long_dev.params()) == abi.WORKSPACE_TOO_SMALL
    # Chunk variant: run() without plan() -> NOT_PLANNED; a short device workspace -> WORKSPACE_TOO_SMALL.
    import ctypes as C

    good = dev.params()
    sizes = session.workspace_sizes(chunk, good)
    import torch

    buf = torch.empty(int(sizes.device_bytes) + 256, dtype=torch.uint8, device="cuda")
    plan = C.create_string_buffer(int(sizes.plan_bytes))
    ws = abi.new(abi.Workspace)
    ws.device = (buf.data_ptr() + 255) // 256 * 256
    ws.device_bytes = sizes.device_bytes
    ws.plan, ws.plan_bytes = C.addressof(plan), sizes.plan_bytes
    assert status(chunk, good, ws) == abi.NOT_PLANNED
    ws.device_bytes = sizes.device_bytes - 256
    assert status(chunk, good, ws) == abi.WORKSPACE_TOO_SMALL
    torch.cuda.synchronize()


def test_recurrent_variant_graph_replays():
    """GRAPH_CAPTURABLE: a mixed call (chunk-routed and token-serial sequences) captured into a graph and replayed
    three times, with eager work between the replays, gives the eager result bit for bit every time."""
    import torch

    rng = np.random.default_rng(29)
    d = cases.make_gdn(rng, [1, 40, 1, 130, 3], 8, slots=[0, 2, 4, 6, 7])
    stream = torch.cuda.Stream()
    session = roost_amd.OpSession(stream=stream)
    try:
        dev = DevGdn(d)
        p = dev.params()
        entry = session.lib.entry(roost_amd.RECURRENT_VARIANT)
        pool0 = dev.pool.clone()
        with torch.cuda.stream(stream):
            session.launch(entry, p, key="graph")  # allocates the workspace outside the capture
        ws = session._ws[(entry.variant_id, "graph")][3]
        stream.synchronize()
        want_o, want_pool = dev.out.clone(), dev.pool.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            session.run(entry, p, ws)
        for replay in range(3):
            with torch.cuda.stream(stream):  # the replay too: replay() launches on the current stream
                dev.pool.copy_(pool0)
                dev.out.fill_(float("nan"))
                graph.replay()
            stream.synchronize()
            assert torch.equal(dev.out.view(torch.int16), want_o.view(torch.int16)), f"replay {replay} output"
            assert torch.equal(dev.pool, want_pool), f"replay {replay} state"
        want_o_np, want_pool_np = cases.oracle_gdn(d)
        cases.assert_close(cases.bf16_values(from_dev(dev.out, True)[: d.tokens]), cases.bf16_values(want_o_np),
                           what="graph output")
    finally:
        session.close()


# ---- Grouped value heads: v_heads = g * k_heads (CpuOps.Hybrid.cs:31-34, 95: value head h reads key head h / g) ------

GROUP_CASES = [
    ("8 key / 16 value heads", 8, 16, [300, 1, 77, 40, 1]),
    ("4 key / 16 value heads", 4, 16, [130, 1, 1, 64]),
    ("16 key / 32 value heads", 16, 32, [200, 1, 1, 20]),
    ("2 key / 16 value heads decode", 2, 16, [1, 1, 1, 1, 1]),
]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("name,kh,vh,lens", GROUP_CASES, ids=[c[0] for c in GROUP_CASES])
def test_grouped_value_heads(session, variant, name, kh, vh, lens):
    import torch

    rng = np.random.default_rng(kh * 100 + vh)
    T, B = int(sum(lens)), len(lens)
    qk_row, v_row = kh * DIM, vh * DIM
    width = 2 * qk_row + v_row  # one fused [q | k | v] row per token, read through strided views
    fused = cases.bf16_bits(rng.standard_normal((T, width), dtype=np.float32))
    g = (-np.logaddexp(0.0, rng.standard_normal((T, vh)))).astype(np.float32)
    beta = cases.bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal((T, vh)))))
    slots_n = B + 2
    pool = (rng.standard_normal((slots_n, vh, DIM, DIM), dtype=np.float32) * 0.05).astype(np.float32)
    slots = rng.permutation(slots_n)[:B].astype(np.int32)  # distinct: sequences of one call never share a slot
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want_o = np.zeros((T, vh, DIM), np.uint16)
    want_pool = pool.copy()
    q, k, v = (np.ascontiguousarray(fused[:, a:b]) for a, b in
               ((0, qk_row), (qk_row, 2 * qk_row), (2 * qk_row, width)))
    oracle.gated_delta_rule(q, k, v, g, beta, want_o, want_pool, slots, cu, batch=B, tokens=T, k_heads=kh, v_heads=vh,
                            k_dim=DIM, v_dim=DIM, l2_norm_qk=True, bf16=True, beta_bf16=True,
                            threads=oracle.host_threads())
    dfused, dpool = to_dev(fused, True), to_dev(pool)
    out = torch.full((T, vh, DIM), float("nan"), dtype=torch.bfloat16, device="cuda")
    reach_qk, reach_v = (T - 1) * width + qk_row, (T - 1) * width + v_row
    p = roost_amd.gated_delta_rule_params(
        dfused, dfused, dfused, to_dev(g), to_dev(beta, True), out, dpool, to_dev(slots), to_dev(cu), batch=B, tokens=T,
        k_heads=kh, v_heads=vh, q_stride=width, k_stride=width, v_stride=width, q_len=reach_qk, k_len=reach_qk,
        v_len=reach_v, q_offset=0, k_offset=qk_row, v_offset=2 * qk_row, cu_seqlens_host=cu)
    session.launch(session.lib.entry(variant), p, key=("group", kh, vh, T))
    got_o, got_pool = from_dev(out, True), from_dev(dpool)
    cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o), what=f"{name} output")
    for s in slots:
        cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"{name} state {s}")


# ---- GatedDeltaRuleGates folded into the recurrent variant (roost_amd_gdn_recurrent_gated_run) ------------------------

GATED_CASES = [
    ("decode 48 x 1", [1] * 48),
    ("routed step 1, 40, 1, 600, 3", [1, 40, 1, 600, 3]),
    ("short continuations", [5, 9, 15, 1]),
]


@pytest.mark.parametrize("name,lens", GATED_CASES, ids=[c[0] for c in GATED_CASES])
def test_recurrent_with_gates_folded_in_equals_gates_then_recurrent(session, name, lens):
    """The fused call against the two calls it replaces, bit for bit (outputs and every state slot): the gates op
    writes g (f32) and beta (bf16) from a [tokens, 64] projection (b at column 0, a at 16, Qwen3.5's layout), then the
    recurrent variant reads them; the fused call reads the projection itself. One case is also checked against CpuOps."""
    import torch

    rng = np.random.default_rng(zlib.crc32(name.encode()))
    d = cases.make_gdn(rng, lens, len(lens) + 3, slots=list(rng.permutation(len(lens) + 3)[: len(lens)]),
                       baseline_style=True)
    T, row = d.tokens, 64
    proj = cases.bf16_bits(rng.standard_normal((T, row)).astype(np.float32) * 4.0)
    a_log = (rng.standard_normal(HEADS) * 0.5).astype(np.float32)
    dt_bias = (rng.standard_normal(HEADS) * 2.0).astype(np.float32)
    d_proj, d_alog, d_dtb = to_dev(proj, True), to_dev(a_log), to_dev(dt_bias)
    reach = (T - 1) * row + HEADS
    gkw = dict(tokens=T, v_heads=HEADS, a_stride=row, b_stride=row, a_len=reach, b_len=reach, a_offset=16, b_offset=0)

    # The two calls: gates into g / beta, then the recurrent variant on them.
    two = DevGdn(d)
    two.g = torch.full((T, HEADS), float("nan"), dtype=torch.float32, device="cuda")
    two.beta = torch.zeros((T, HEADS), dtype=torch.bfloat16, device="cuda")
    roost_amd.gated_delta_rule_gates(session, d_proj, d_proj, d_alog, d_dtb, two.g, two.beta, **gkw)
    session.launch(session.lib.entry(roost_amd.RECURRENT_VARIANT), two.params(), key=("gated-two", T))
    torch.cuda.synchronize()
    want_o, want_pool = from_dev(two.out, True)[:T], from_dev(two.pool)

    # The fused call: g and beta spans left empty.
    one = DevGdn(d)
    one.g = None
    one.beta = None
    gates = roost_amd.gated_delta_rule_gates_params(d_proj, d_proj, d_alog, d_dtb, None, None, **gkw)
    roost_amd.gdn_recurrent_gated(session, one.params(), gates, key=("gated-one", T))
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(one.out, True)[:T], want_o), "outputs differ from gates + recurrent"
    assert np.array_equal(from_dev(one.pool), want_pool), "states differ from gates + recurrent"

    if name.startswith("routed"):
        d.g = np.ascontiguousarray(from_dev(two.g).reshape(T, HEADS))
        d.beta = np.ascontiguousarray(from_dev(two.beta, True).reshape(T, HEADS))
        want_o_cpu, want_pool_cpu = cases.oracle_gdn(d)
        cases.assert_close(cases.bf16_values(want_o), cases.bf16_values(want_o_cpu), what="fused gates vs CpuOps")
        for s in d.slots:
            cases.assert_close(want_pool[s], want_pool_cpu[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"slot {s}")


def test_recurrent_with_gates_refusals(session):
    rng = np.random.default_rng(5)
    d = cases.make_gdn(rng, [1, 1], 2)
    dev = DevGdn(d)
    proj = to_dev(cases.bf16_bits(rng.standard_normal((2, 64)).astype(np.float32)), True)
    vec = to_dev(np.zeros(HEADS, np.float32))
    entry_fn = session.lib.dll.roost_amd_gdn_recurrent_gated_run
    ws = abi.new(abi.Workspace)

    def status(gates, **over):
        import ctypes as C

        params = dev.params(**over)  # held here: the call reads it through a raw address
        return entry_fn(session.ctx, C.addressof(params), C.addressof(gates) if gates is not None else None,
                        C.addressof(ws), C.c_void_p(session.stream_handle))

    good = roost_amd.gated_delta_rule_gates_params(proj, proj, vec, vec, None, None, tokens=2, v_heads=HEADS,
                                                   a_stride=64, b_stride=64, a_offset=16)
    assert status(None) == abi.INVALID_ARGUMENT
    bad = roost_amd.gated_delta_rule_gates_params(proj, proj, vec, vec, None, None, tokens=3, v_heads=HEADS,
                                                  a_stride=64, b_stride=64, a_offset=16)
    assert status(bad) == abi.INVALID_ARGUMENT  # the gates cover another token count
    short = roost_amd.gated_delta_rule_gates_params(proj, proj, vec, vec, None, None, tokens=2, v_heads=HEADS,
                                                    a_stride=64, b_stride=64, a_offset=16, a_len=10)
    assert status(short) == abi.INVALID_ARGUMENT  # a shorter than its view
    assert status(good) == abi.OK


def test_chunk_long_sequence_two_calls_equal_one(session):
    """A size-independent property at a length the oracle cannot reach in a test (two sequences of 131,072 tokens on
    the chunk variant): running each sequence's first half and then its second half in a second call that starts from
    the state the first wrote gives the same outputs and final states, bit for bit, as one call over the whole
    sequences (the halves end on chunk boundaries, so both runs do the same arithmetic). The reference states the same
    invariant on short sequences (HybridTests.cs:174-200)."""
    import torch

    H, D, L, B = 4, DIM, 1 << 17, 2
    g_ = torch.Generator(device="cuda").manual_seed(31)
    fused = (torch.randn((B * L, 3 * H * D), generator=g_, device="cuda") * 0.5).to(torch.bfloat16)
    gg = -torch.nn.functional.softplus(torch.randn((B * L, H), generator=g_, device="cuda")) * 0.05
    beta = torch.sigmoid(torch.randn((B * L, H), generator=g_, device="cuda")).to(torch.bfloat16)
    s0 = torch.randn((B, H, D, D), generator=g_, device="cuda") * 0.01
    slots = torch.arange(B, dtype=torch.int32, device="cuda")
    entry = session.lib.entry(roost_amd.CHUNK_VARIANT)

    def call(rows, lens, pool, out, key):
        cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        tokens = int(cu_h[-1])
        x = fused[rows]
        reach = (tokens - 1) * 3 * H * D + H * D
        p = roost_amd.gated_delta_rule_params(
            x, x, x, gg[rows], beta[rows], out, pool, slots, torch.from_numpy(cu_h).cuda(), batch=B, tokens=tokens,
            k_heads=H, v_heads=H, q_stride=3 * H * D, k_stride=3 * H * D, v_stride=3 * H * D, q_len=reach,
            k_len=reach, v_len=reach, q_offset=0, k_offset=H * D, v_offset=2 * H * D, cu_seqlens_host=cu_h)
        session.launch(entry, p, key=key)

    # One call: sequence b is rows [b L, (b + 1) L).
    pool_one = s0.clone()
    out_one = torch.full((B * L, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    call(slice(None), [L, L], pool_one, out_one, "long-one")
    # Two calls: the first halves of both sequences, then the second halves (rows gathered so each call's sequences
    # are contiguous).
    half = L // 2
    first = torch.cat([torch.arange(b * L, b * L + half) for b in range(B)]).cuda()
    second = torch.cat([torch.arange(b * L + half, (b + 1) * L) for b in range(B)]).cuda()
    pool_two = s0.clone()
    out_a = torch.full((B * half, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    out_b = torch.full((B * half, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    call(first, [half, half], pool_two, out_a, "long-a")
    call(second, [half, half], pool_two, out_b, "long-b")
    torch.cuda.synchronize()
    out_two = torch.empty_like(out_one)
    out_two[first] = out_a
    out_two[second] = out_b
    assert not torch.isnan(out_one.float()).any()
    assert torch.equal(pool_one, pool_two), "final states differ between one call and two"
    assert torch.equal(out_one.view(torch.int16), out_two.view(torch.int16)), "outputs differ between one call and two"


# ---- seeded random calls -------------------------------------------------------------------------------------------

def _random_gdn_case(rng):
    """One call's shape: head counts and groups, fused or separate rows, lengths mixing empty, decode, the 16-token
    routing edge, chunk edges and long sequences, init, scale, decay distribution and, for the recurrent variant,
    whether the host copy of cu_seqlens is given (without it the device routes the call itself)."""
    kh = int(rng.choice([2, 4, 8, 16]))
    vh = kh * int(rng.choice([1, 2, 4]))
    pool_lens = [0, 1, 1, 1, 2, 7, 15, 16, 17, 33, 63, 64, 65, 127, 128, 129, 200, 300, 511]
    lens = [int(rng.choice(pool_lens)) for _ in range(int(rng.integers(1, 9)))]
    if rng.random() < 0.3:
        lens = [1] * int(rng.integers(1, 80))  # a decode step
    c = dict(kh=kh, vh=vh, lens=lens, fused=bool(rng.random() < 0.6), init=bool(rng.random() < 0.8),
             scale=float(rng.choice([0.0, 0.0, 0.05, 0.3])), baseline_style=bool(rng.random() < 0.5),
             host_cu=bool(rng.random() < 0.7), variant=VARIANTS[int(rng.integers(0, 2))])
    if c["variant"] == roost_amd.CHUNK_VARIANT:
        c["host_cu"] = True  # the chunk variant's plan() reads the host copy
    return c


@pytest.mark.parametrize("seed", range(32))
def test_random_gdn_calls_match_cpuops(session, seed):
    """Seeded random calls of either variant against CpuOps' GatedDeltaRule (CpuOps.Hybrid.cs:30-157): outputs to the
    bf16 bar, every owned state slot to the 1e-3 state bar, every other slot untouched."""
    import torch

    rng = np.random.default_rng(5000 + seed)
    c = _random_gdn_case(rng)
    kh, vh, lens = c["kh"], c["vh"], c["lens"]
    T, B = int(sum(lens)), len(lens)
    qk_row, v_row = kh * DIM, vh * DIM
    width = 2 * qk_row + v_row
    fused = cases.bf16_bits(rng.standard_normal((max(T, 1), width), dtype=np.float32))
    if c["baseline_style"]:
        g = (-np.logaddexp(0.0, rng.standard_normal((max(T, 1), vh)))).astype(np.float32)
        beta = cases.bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal((max(T, 1), vh)))))
    else:
        g = (-rng.random((max(T, 1), vh)) * 0.2).astype(np.float32)
        beta = cases.bf16_bits(rng.random((max(T, 1), vh)).astype(np.float32))
    slots_n = B + 3
    pool = (rng.standard_normal((slots_n, vh, DIM, DIM), dtype=np.float32) * 0.05).astype(np.float32)
    slots = rng.permutation(slots_n)[:B].astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v = (np.ascontiguousarray(fused[:, a:b]) for a, b in
               ((0, qk_row), (qk_row, 2 * qk_row), (2 * qk_row, width)))
    want_o = np.zeros((max(T, 1), vh, DIM), np.uint16)
    want_pool = pool.copy()
    oracle.gated_delta_rule(q, k, v, g, beta, want_o, want_pool, slots, cu, batch=B, tokens=T, k_heads=kh, v_heads=vh,
                            k_dim=DIM, v_dim=DIM, use_initial_state=c["init"], l2_norm_qk=True, scale=c["scale"],
                            bf16=True, beta_bf16=True, threads=oracle.host_threads())
    dpool = to_dev(pool)
    out = torch.full((max(T, 1), vh, DIM), float("nan"), dtype=torch.bfloat16, device="cuda")
    common = dict(batch=B, tokens=T, k_heads=kh, v_heads=vh, use_initial_state=c["init"], scale=c["scale"],
                  cu_seqlens_host=cu if c["host_cu"] else None)
    if c["fused"]:
        dfused = to_dev(fused, True)
        reach_qk = 0 if T == 0 else (T - 1) * width + qk_row
        reach_v = 0 if T == 0 else (T - 1) * width + v_row
        p = roost_amd.gated_delta_rule_params(
            dfused, dfused, dfused, to_dev(g), to_dev(beta, True), out, dpool, to_dev(slots), to_dev(cu),
            q_stride=width, k_stride=width, v_stride=width, q_len=reach_qk, k_len=reach_qk, v_len=reach_v,
            q_offset=0, k_offset=qk_row, v_offset=2 * qk_row, **common)
    else:
        p = roost_amd.gated_delta_rule_params(to_dev(q, True), to_dev(k, True), to_dev(v, True), to_dev(g),
                                              to_dev(beta, True), out, dpool, to_dev(slots), to_dev(cu), **common)
    print(f"seed {seed}: {c}", flush=True)
    session.launch(session.lib.entry(c["variant"]), p, key=("random", seed))
    got_o, got_pool = from_dev(out, True)[:T], from_dev(dpool)
    cases.assert_close(cases.bf16_values(got_o), cases.bf16_values(want_o[:T]), what=f"seed {seed} output")
    owned = {int(slots[b]) for b in range(B) if lens[b] > 0}
    for s in range(slots_n):
        if s in owned:
            cases.assert_close(got_pool[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL,
                               what=f"seed {seed} state {s}")
        else:
            assert got_pool[s].tobytes() == pool[s].tobytes(), f"seed {seed}: slot {s} was touched"
