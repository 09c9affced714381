"""Seeded random calls of the three fused GDN-layer entry points (roost_amd_gdn_decode_layer_run, roost_amd_gdn_layer_run
and roost_amd_gdn_chunk_layer_run) against the four ops they replace (CausalConv1d, GatedDeltaRuleGates, GatedDeltaRule,
GatedRmsNorm; Qwen35EagerModel.cs:89-92 runs them one after another), bit for bit: norm output, every recurrent state
slot and every convolution state slot. Each of the four ops is checked against the CpuOps oracle in its own tests."""
import numpy as np
import pytest

import cases
from test_attention_gpu import from_dev
from test_gdn_chunk_layer_gpu import ChunkLayer
from test_gdn_decode_layer_gpu import Layer
import roost_amd

pytestmark = pytest.mark.gpu

KINDS = ("decode", "any", "chunk")


def _random_layer_case(rng, kind):
    kh = int(rng.choice([1, 2, 4, 8, 16]))
    vh = kh * int(rng.choice([1, 2, 4]))
    if kind == "decode":  # every sequence under the 16-token routing edge
        lens = [int(rng.choice([0, 1, 1, 1, 2, 5, 15])) for _ in range(int(rng.integers(1, 40)))]
    else:
        lens = [int(rng.choice([0, 1, 1, 3, 15, 16, 17, 63, 64, 65, 130, 257])) for _ in range(int(rng.integers(1, 8)))]
    B = len(lens)
    n_slots = B + 2
    unslot = kind != "any" and rng.random() < 0.4

    def slots():
        s = rng.permutation(n_slots)[:B].astype(np.int32)
        if unslot:
            s[rng.random(B) < 0.25] = -1
        return [int(v) for v in s]

    return dict(lens=lens, kh=kh, vh=vh, width=int(rng.integers(1, 5)), bias=bool(rng.random() < 0.6),
                sdt=str(rng.choice(["bf16", "f32"])), fg=bool(rng.random() < 0.6), slots=slots(), cslots=slots(),
                cu_host=kind != "any" or bool(rng.random() < 0.7))


@pytest.mark.parametrize("seed", range(24))
def test_random_layer_calls_equal_the_four_ops(session, seed):
    kind = KINDS[seed % 3]
    rng = np.random.default_rng(7000 + seed)
    c = _random_layer_case(rng, kind)
    print(f"seed {seed} {kind}: {c}", flush=True)
    cls = ChunkLayer if kind == "chunk" else Layer
    layer = cls(rng, c["lens"], c["kh"], c["vh"], c["width"], c["bias"], c["sdt"], c["fg"], c["slots"], c["cslots"])
    T = layer.T * layer.vh
    if kind == "chunk":
        want = layer.four_ops(session)
        got = layer.fused(session)
        for what in want:
            assert np.array_equal(got[what], want[what]), f"seed {seed}: {what} differs from the four ops"
        out = got["norm output"]
    else:
        want_out, want_cs, want_st = layer.four_ops(session)
        t = layer.t
        if kind == "decode":
            out, cs, st = layer.fused(session)
        else:
            y, o, dout, dcs, dst = layer.buffers()
            gates = layer.gates_params(None, None) if c["fg"] else None
            gdn = layer.gdn_params(y, o, dst, None if c["fg"] else layer.g, None if c["fg"] else layer.beta,
                                   cu_host=c["cu_host"])
            roost_amd.gdn_layer(session, layer.conv_params(y, dcs), gates, gdn, layer.norm_params(o, dout),
                                key=("random", seed))
            t.cuda.synchronize()
            out, cs, st = from_dev(dout, True), from_dev(dcs, dcs.dtype == t.bfloat16), from_dev(dst)
        assert np.array_equal(out[:T], want_out[:T]), f"seed {seed}: norm output differs from the four ops"
        assert np.array_equal(cs, want_cs), f"seed {seed}: convolution states differ from the four ops"
        assert np.array_equal(st, want_st), f"seed {seed}: recurrent states differ from the four ops"
    assert not np.isnan(cases.bf16_values(out[:T])).any()
