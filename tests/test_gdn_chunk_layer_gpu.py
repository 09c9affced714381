"""roost_amd_gdn_chunk_layer_run: one prefill pass of a Gated DeltaNet layer over the chunk variant (CausalConv1d,
GatedDeltaRuleGates, the chunked GatedDeltaRule and GatedRmsNorm; Qwen35EagerModel.cs:89-92 runs them one after
another), with the convolution folded into the chunk prep. Each case runs the four ops through their own entry points
(the chunk variant for the GDN op) and the layer call on copies of the same states, and requires the convolution's
output, the GDN output, the norm's output, every recurrent state slot and every convolution state slot to match bit for
bit. Each of the four ops is checked against the CpuOps oracle in its own tests; equality with them is the parity claim
here."""
import zlib

import numpy as np
import pytest

import cases
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev, torch
from test_gdn_decode_layer_gpu import Layer

pytestmark = pytest.mark.gpu

# (name, sequence lengths, k_heads, v_heads, width, bias, conv state dtype, gates folded in, GDN slots, conv slots)
CHUNK_LAYER_CASES = [
    ("two 300-token prefills, a full chunk, a decode row", [300, 64, 1, 300], 16, 16, 4, True, "bf16", True, None,
     None),
    ("short sequences and an empty row (state in every tap)", [2, 0, 3, 1, 70], 4, 4, 4, False, "f32", False, None,
     None),
    ("group 2, width 3, unslotted rows", [129, 5, 64, 200], 4, 8, 3, True, "bf16", True, [0, -1, 2, 3],
     [3, 2, -1, 0]),
    ("width 2, one head", [65, 1, 127], 1, 1, 2, True, "f32", True, None, None),
]


class ChunkLayer(Layer):
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
        session.launch(session.lib.entry(roost_amd.CHUNK_VARIANT), self.gdn_params(y, o, st, g, beta),
                       key=("chunk-four", self.B, self.T))
        session.launch(session.lib.entry(roost_amd.GATED_RMS_NORM_VARIANT), self.norm_params(o, out))
        t.cuda.synchronize()
        return self.result(y, o, out, cs, st)

    def fused(self, session, cu_host=True, plan=True):
        t = self.t
        y, o, out, cs, st = self.buffers()
        gates = self.gates_params(None, None) if self.fused_gates else None
        gdn = self.gdn_params(y, o, st, None if self.fused_gates else self.g, None if self.fused_gates else self.beta,
                              cu_host=cu_host)
        roost_amd.gdn_chunk_layer(session, self.conv_params(y, cs), gates, gdn, self.norm_params(o, out),
                                  key=(self.B, self.T), plan=plan)
        t.cuda.synchronize()
        return self.result(y, o, out, cs, st)

    def result(self, y, o, out, cs, st):
        t = self.t
        return {"conv output": from_dev(y, True)[: self.T], "GDN output": from_dev(o, True)[: self.T],
                "norm output": from_dev(out, True)[: self.T * self.vh],
                "convolution states": from_dev(cs, cs.dtype == t.bfloat16), "recurrent states": from_dev(st)}


@pytest.mark.parametrize("name,lens,kh,vh,width,bias,sdt,fg,slots,cslots", CHUNK_LAYER_CASES,
                         ids=[c[0] for c in CHUNK_LAYER_CASES])
def test_chunk_layer_equals_the_four_ops(session, name, lens, kh, vh, width, bias, sdt, fg, slots, cslots):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = ChunkLayer(rng, lens, kh, vh, width, bias, sdt, fg, slots, cslots)
    want = layer.four_ops(session)
    got = layer.fused(session)
    for what in want:
        assert np.array_equal(got[what], want[what]), f"{what} differs from the four ops"
    assert not np.isnan(cases.bf16_values(got["norm output"])).any()
    # Repeatable, and run() reads no host table: a second call on the same plan without cu_seqlens_host gives the same
    # bits.
    again = layer.fused(session, cu_host=False, plan=False)
    assert np.array_equal(again["norm output"], got["norm output"])


def test_chunk_layer_refusals(session):
    t = torch()
    rng = np.random.default_rng(29)
    layer = ChunkLayer(rng, [70, 3], 2, 2, 4, True, "bf16", True, None, None)
    y, o, out, cs, st = layer.buffers()

    def status(conv=None, gdn=None, norm=None, plan=True):
        conv = conv if conv is not None else layer.conv_params(y, cs)
        gdn = gdn if gdn is not None else layer.gdn_params(y, o, st)
        norm = norm if norm is not None else layer.norm_params(o, out)
        try:
            roost_amd.gdn_chunk_layer(session, conv, layer.gates_params(None, None), gdn, norm, key="refusals",
                                      plan=plan)
        except roost_amd.KernelError as e:
            return e.status
        return abi.OK

    assert status() == abi.OK
    assert status(gdn=layer.gdn_params(t.empty_like(y), o, st)) == abi.INVALID_ARGUMENT  # q/k/v not conv-output views
    assert status(norm=layer.norm_params(t.empty_like(o), out)) == abi.INVALID_ARGUMENT  # the norm does not read o
    wide = ChunkLayer(rng, [70, 3], 2, 2, 5, True, "bf16", True, None, None)
    wy, wo, wout, wcs, wst = wide.buffers()
    with pytest.raises(roost_amd.KernelError) as e:
        roost_amd.gdn_chunk_layer(session, wide.conv_params(wy, wcs), wide.gates_params(None, None),
                                  wide.gdn_params(wy, wo, wst), wide.norm_params(wo, wout), key="wide")
    assert e.value.status == abi.UNSUPPORTED
    # A workspace planned for another batch is NOT_PLANNED.
    other = ChunkLayer(rng, [10, 3], 2, 2, 4, True, "bf16", True, None, None)
    oy, oo, oout, ocs, ost = other.buffers()
    roost_amd.gdn_chunk_layer(session, other.conv_params(oy, ocs), other.gates_params(None, None),
                              other.gdn_params(oy, oo, ost), other.norm_params(oo, oout), key="replan")
    with pytest.raises(roost_amd.KernelError) as e:
        roost_amd.gdn_chunk_layer(session, layer.conv_params(y, cs), layer.gates_params(None, None),
                                  layer.gdn_params(y, o, st), layer.norm_params(o, out), key="replan", plan=False)
    assert e.value.status == abi.NOT_PLANNED
