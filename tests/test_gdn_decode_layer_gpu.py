"""roost_amd_gdn_decode_layer_run: one decode step of a Gated DeltaNet layer (CausalConv1d, GatedDeltaRuleGates, the
recurrent GatedDeltaRule and GatedRmsNorm; Qwen35EagerModel.cs:89-92 runs them one after another) in one call. Each
case runs the four ops through their own entry points and the fused call on copies of the same states, and requires
the norm's output, every recurrent state slot and every convolution state slot to match bit for bit. Each of the four
ops is checked against the CpuOps oracle in its own tests; equality with them is the parity claim here."""
import zlib

import numpy as np
import pytest

import cases
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev, to_dev, torch

pytestmark = pytest.mark.gpu

DIM = 128

# (name, sequence lengths, k_heads, v_heads, width, bias, conv state dtype, gates folded in, GDN slots, conv slots)
LAYER_CASES = [
    ("decode 48 x 1 (Qwen3.5 0.8B)", [1] * 48, 16, 16, 4, True, "bf16", True, None, None),
    ("short continuations and an empty row", [5, 0, 15, 1, 3], 16, 16, 4, False, "f32", False, None, None),
    ("group 2, width 3, unslotted rows", [1] * 10, 8, 16, 3, True, "bf16", True,
     [0, -1, 2, 3, 4, 5, 6, 7, 8, 9], [9, 8, 7, -1, 5, 4, 3, 2, 1, 0]),
    ("width 2, two heads", [2, 1, 4], 2, 2, 2, True, "f32", True, None, None),
    # Sequences sharing a recurrent state slot run in batch order, as the recurrent variant (and CpuOps) runs them.
    ("shared state slots in batch order", [1, 3, 0, 1, 2, 1], 4, 8, 4, True, "bf16", True, [3, 3, 3, 1, 3, 1],
     [0, 1, 2, 3, 4, 5]),
    ("width 1", [1, 2, 1], 2, 4, 1, False, "bf16", False, None, None),
]


class Layer:
    """A decode layer's inputs and states on the device, and its calls (the four ops, or the fused one)."""

    def __init__(self, rng, lens, kh, vh, width, bias, state_dtype, fused_gates, slots, conv_slots):
        t = torch()
        self.lens, self.kh, self.vh, self.width = lens, kh, vh, width
        self.B, self.T = len(lens), int(sum(lens))
        self.ch = 2 * kh * DIM + vh * DIM
        self.cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        self.cu = to_dev(self.cu_h)
        n_slots = self.B + 2
        self.slots = to_dev(np.array(slots if slots is not None else rng.permutation(n_slots)[: self.B], np.int32))
        self.cslots = to_dev(np.array(conv_slots if conv_slots is not None else rng.permutation(n_slots)[: self.B],
                                      np.int32))
        bf = lambda a: to_dev(cases.bf16_bits(a.astype(np.float32)), True)  # noqa: E731
        T, ch = self.T, self.ch
        self.x = bf(rng.standard_normal((max(T, 1), ch)))
        self.w = bf(rng.standard_normal((ch, width)) * 0.5)
        self.bias = bf(rng.standard_normal(ch) * 0.3) if bias else None
        sw = max(width - 1, 1)
        cs = rng.standard_normal((n_slots, ch, sw)).astype(np.float32)
        self.conv_state = bf(cs) if state_dtype == "bf16" else to_dev(cs)
        self.state = to_dev((rng.standard_normal((n_slots, vh, DIM, DIM)) * 0.01).astype(np.float32))
        self.fused_gates = fused_gates
        self.proj = bf(rng.standard_normal((max(T, 1), 2 * vh)) * 3.0)
        self.a_log = to_dev((rng.standard_normal(vh) * 0.5).astype(np.float32))
        self.dt_bias = to_dev((rng.standard_normal(vh) * 2.0).astype(np.float32))
        gl = -np.log1p(np.exp(rng.standard_normal((max(T, 1), vh))))
        self.g = to_dev(gl.astype(np.float32))
        self.beta = bf(1.0 / (1.0 + np.exp(-rng.standard_normal((max(T, 1), vh)))))
        self.z = bf(rng.standard_normal((max(T, 1) * vh, DIM)) * 2.0)
        self.norm_w = to_dev((1.0 + rng.standard_normal(DIM) * 0.2).astype(np.float32))
        self.eps = 1e-6
        self.t = t

    def buffers(self):
        t = self.t
        T = max(self.T, 1)
        y = t.full((T, self.ch), float("nan"), dtype=t.bfloat16, device="cuda")
        o = t.full((T, self.vh, DIM), float("nan"), dtype=t.bfloat16, device="cuda")
        out = t.full((T * self.vh, DIM), float("nan"), dtype=t.bfloat16, device="cuda")
        return y, o, out, self.conv_state.clone(), self.state.clone()

    def conv_params(self, y, cs):
        return roost_amd.causal_conv1d_params(self.x, self.w, self.bias, y, cs, self.cslots, self.cu, batch=self.B,
                                              tokens=self.T, channels=self.ch, width=self.width, silu=True)

    def gdn_params(self, y, o, state, g=None, beta=None, cu_host=True):
        qk, T = self.kh * DIM, max(self.T, 1)
        reach_qk, reach_v = (T - 1) * self.ch + qk, (T - 1) * self.ch + self.vh * DIM
        return roost_amd.gated_delta_rule_params(
            y, y, y, g, beta, o, state, self.slots, self.cu, batch=self.B, tokens=self.T, k_heads=self.kh,
            v_heads=self.vh, q_stride=self.ch, k_stride=self.ch, v_stride=self.ch, q_len=reach_qk, k_len=reach_qk,
            v_len=reach_v, q_offset=0, k_offset=qk, v_offset=2 * qk, cu_seqlens_host=self.cu_h if cu_host else None)

    def gates_params(self, g, beta):
        reach = (max(self.T, 1) - 1) * 2 * self.vh + self.vh
        return roost_amd.gated_delta_rule_gates_params(
            self.proj, self.proj, self.a_log, self.dt_bias, g, beta, tokens=self.T, v_heads=self.vh,
            a_stride=2 * self.vh, b_stride=2 * self.vh, a_len=reach, b_len=reach, a_offset=self.vh, b_offset=0)

    def norm_params(self, o, out):
        return roost_amd.gated_rms_norm_params(o, self.z, self.norm_w, out, rows=self.T * self.vh, dim=DIM,
                                               eps=self.eps)

    def four_ops(self, session):
        t = self.t
        y, o, out, cs, st = self.buffers()
        roost_amd.causal_conv1d(session, self.x, self.w, self.bias, y, cs, self.cslots, self.cu, batch=self.B,
                                tokens=self.T, channels=self.ch, width=self.width, silu=True)
        g, beta = self.g, self.beta
        if self.fused_gates:
            g = t.full((max(self.T, 1), self.vh), float("nan"), dtype=t.float32, device="cuda")
            beta = t.zeros((max(self.T, 1), self.vh), dtype=t.bfloat16, device="cuda")
            session.launch(session.lib.entry(roost_amd.GATES_VARIANT), self.gates_params(g, beta))
        p = self.gdn_params(y, o, st, g, beta)
        session.launch(session.lib.entry(roost_amd.RECURRENT_VARIANT), p, key=("layer-four", self.B, self.T))
        session.launch(session.lib.entry(roost_amd.GATED_RMS_NORM_VARIANT), self.norm_params(o, out))
        t.cuda.synchronize()
        return from_dev(out, True), from_dev(cs, cs.dtype == t.bfloat16), from_dev(st)

    def fused(self, session):
        t = self.t
        y, o, out, cs, st = self.buffers()
        gates = self.gates_params(None, None) if self.fused_gates else None
        gdn = self.gdn_params(y, o, st, None if self.fused_gates else self.g, None if self.fused_gates else self.beta)
        roost_amd.gdn_decode_layer(session, self.conv_params(y, cs), gates, gdn, self.norm_params(o, out))
        t.cuda.synchronize()
        return from_dev(out, True), from_dev(cs, cs.dtype == t.bfloat16), from_dev(st)


@pytest.mark.parametrize("name,lens,kh,vh,width,bias,sdt,fg,slots,cslots", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_decode_layer_equals_the_four_ops(session, name, lens, kh, vh, width, bias, sdt, fg, slots, cslots):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = Layer(rng, lens, kh, vh, width, bias, sdt, fg, slots, cslots)
    want_out, want_cs, want_st = layer.four_ops(session)
    got_out, got_cs, got_st = layer.fused(session)
    T = layer.T * vh
    assert np.array_equal(got_out[:T], want_out[:T]), "norm output differs from the four ops"
    assert np.array_equal(got_cs, want_cs), "convolution states differ from the four ops"
    assert np.array_equal(got_st, want_st), "recurrent states differ from the four ops"
    assert not np.isnan(cases.bf16_values(got_out[:T])).any()
    # The call is repeatable: a second fused call from the same starting states gives the same bits.
    again_out, _, _ = layer.fused(session)
    assert np.array_equal(again_out[:T], got_out[:T])


def test_decode_layer_refusals(session):
    t = torch()
    rng = np.random.default_rng(17)
    layer = Layer(rng, [1, 1, 1], 16, 16, 4, True, "bf16", True, None, None)
    y, o, out, cs, st = layer.buffers()

    def status(conv=None, gates="default", gdn=None, norm=None):
        conv = conv if conv is not None else layer.conv_params(y, cs)
        gates = layer.gates_params(None, None) if gates == "default" else gates
        gdn = gdn if gdn is not None else layer.gdn_params(y, o, st)
        norm = norm if norm is not None else layer.norm_params(o, out)
        try:
            roost_amd.gdn_decode_layer(session, conv, gates, gdn, norm)
        except roost_amd.KernelError as e:
            return e.status
        return abi.OK

    assert status() == abi.OK
    assert status(gdn=layer.gdn_params(y, o, st, cu_host=False)) == abi.INVALID_ARGUMENT
    other = t.empty_like(y)
    assert status(gdn=layer.gdn_params(other, o, st)) == abi.INVALID_ARGUMENT  # q/k/v not views of the conv output
    assert status(norm=layer.norm_params(t.empty_like(o), out)) == abi.INVALID_ARGUMENT  # norm input is not o
    assert status(norm=roost_amd.gated_rms_norm_params(o, layer.z, layer.norm_w, layer.x, rows=3 * 16, dim=DIM,
                                                       eps=1e-6)) == abi.INVALID_ARGUMENT  # output over the conv input
    wide = Layer(rng, [1, 1, 1], 16, 16, 5, True, "bf16", True, None, None)
    wy, wo, wout, wcs, wst = wide.buffers()
    with pytest.raises(roost_amd.KernelError) as e:
        roost_amd.gdn_decode_layer(session, wide.conv_params(wy, wcs), wide.gates_params(None, None),
                                   wide.gdn_params(wy, wo, wst), wide.norm_params(wo, wout))
    assert e.value.status == abi.UNSUPPORTED
    long = Layer(rng, [16, 1], 16, 16, 4, True, "bf16", True, None, None)
    ly, lo, lout, lcs, lst = long.buffers()
    with pytest.raises(roost_amd.KernelError) as e:
        roost_amd.gdn_decode_layer(session, long.conv_params(ly, lcs), long.gates_params(None, None),
                                   long.gdn_params(ly, lo, lst), long.norm_params(lo, lout))
    assert e.value.status == abi.UNSUPPORTED
    # Nothing was written by the refused calls.
    assert np.array_equal(from_dev(lst), from_dev(long.state))


def test_decode_layer_empty_step(session):
    """A step whose sequences are all empty reads and writes nothing, as the four ops do."""
    rng = np.random.default_rng(23)
    layer = Layer(rng, [0, 0], 16, 16, 4, True, "bf16", True, None, None)
    out, cs, st = layer.fused(session)
    assert np.array_equal(cs, from_dev(layer.conv_state, True))
    assert np.array_equal(st, from_dev(layer.state))


# roost_amd_gdn_layer_run: the same layer for any step over the recurrent variant (the decode-layer kernel when every
# sequence is short, else the conv op, the recurrent variant with the gates folded in and the norm op).
ANY_LAYER_CASES = [
    ("decode 16 x 1 (decode-layer kernel)", [1] * 16, 16, 16, 4, True, "bf16", True, True),
    ("mixed step: prefills beside decode rows", [1, 600, 17, 0, 3, 1, 64], 16, 16, 4, True, "bf16", True, True),
    ("mixed step, group 2, width 3, f32 state, g and beta read", [200, 1, 1, 40], 8, 16, 3, False, "f32", False, True),
    ("no host lengths (device routing)", [1, 30, 2, 16], 4, 4, 4, True, "bf16", True, False),
]


@pytest.mark.parametrize("name,lens,kh,vh,width,bias,sdt,fg,cu_host", ANY_LAYER_CASES,
                         ids=[c[0] for c in ANY_LAYER_CASES])
def test_any_step_layer_equals_the_four_ops(session, name, lens, kh, vh, width, bias, sdt, fg, cu_host):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = Layer(rng, lens, kh, vh, width, bias, sdt, fg, None, None)
    want_out, want_cs, want_st = layer.four_ops(session)
    t = layer.t
    y, o, out, cs, st = layer.buffers()
    gates = layer.gates_params(None, None) if fg else None
    gdn = layer.gdn_params(y, o, st, None if fg else layer.g, None if fg else layer.beta, cu_host=cu_host)
    roost_amd.gdn_layer(session, layer.conv_params(y, cs), gates, gdn, layer.norm_params(o, out), key=name)
    t.cuda.synchronize()
    T = layer.T * vh
    assert np.array_equal(from_dev(out, True)[:T], want_out[:T]), "norm output differs from the four ops"
    assert np.array_equal(from_dev(cs, cs.dtype == t.bfloat16), want_cs), "convolution states differ from the four ops"
    assert np.array_equal(from_dev(st), want_st), "recurrent states differ from the four ops"
    assert not np.isnan(cases.bf16_values(from_dev(out, True)[:T])).any()
