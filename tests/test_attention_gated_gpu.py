"""roost_amd_paged_attention_gated_run: PagedAttention with Qwen3.5's output gate (SigmoidMul, CpuOps.Gating.cs:84-96)
folded into the kernels that write the output. The reference's worker runs the two ops one after the other
(Qwen35EagerModel.cs:94-97); the fused call must give the same bits, which each case checks against run() followed by
the SigmoidMul op on the GPU, for every kernel that writes output rows: decode (bf16 and f32, whole rows and split rows
merged), the prefill tile kernel (whole items and split pieces merged in both merge forms), the general prefill kernel
(page size 7), the f32 prefill rows, and config 5's mixed step, whose decode rows run in the same launch as its tile pieces.
The ungated attention itself is checked against the oracle elsewhere; here the gate is also shown to change the output,
and the lse output to be the ungated one."""
import zlib

import numpy as np
import pytest

import cases
import roost_amd
from roost_amd import abi
from test_attention_gpu import Dev, from_dev, to_dev, torch

pytestmark = pytest.mark.gpu

# (name, [(q_len, kv_len)], page_size, hnd, causal, window, head_dim, bf16)
GATED_CASES = [
    ("decode mixed8 (split rows merged)", [(1, 900), (1, 17), (1, 1), (1, 2048), (1, 333), (1, 64), (1, 1024), (1, 777)],
     16, False, True, -1, 256, True),
    ("decode single 6000 HND ps64", [(1, 6000)], 64, True, True, -1, 256, True),
    ("decode f32 hd128", [(1, 5), (1, 37), (1, 1300)], 16, False, True, -1, 128, False),
    ("prefill tile split and merged", [(128, 8000), (64, 2000), (200, 1200), (64, 64)], 16, False, True, -1, 256, True),
    ("prefill tile hd128 window", [(300, 2500), (37, 300)], 16, False, True, 200, 128, True),
    ("prefill general page size 7", [(100, 300), (33, 33)], 7, False, True, -1, 256, True),
    ("prefill f32 rows", [(37, 300), (1, 90), (6, 9000)], 16, False, True, -1, 256, False),
    ("mixed step non-causal", [(1, 900), (100, 300), (1, 45)], 16, False, False, -1, 256, True),
]


def _gate(rng, out, bf16):
    g = (rng.standard_normal(out.shape) * 2.0).astype(np.float32)
    return to_dev(cases.bf16_bits(g) if bf16 else g, bf16)


def _check(session, b, causal=True, window=-1, key="gated"):
    rng = np.random.default_rng(zlib.crc32(key.encode()))
    t = torch()
    d = Dev(b, causal, with_lse=True, window_left=window)
    entry = session.lib.entry(roost_amd.ATTENTION_VARIANT)
    p = d.params()
    session.launch(entry, p, key=(key, "plain"))
    plain = from_dev(d.out, b.bf16).copy()
    plain_lse = from_dev(d.lse).copy()
    gate = _gate(rng, plain, b.bf16)
    rows, dim = b.tokens, b.hq * b.d
    # run() then the SigmoidMul op on its output, in place (how the worker applies the gate).
    roost_amd.sigmoid_mul(session, d.out, gate, d.out, rows=rows, dim=dim)
    want = from_dev(d.out, b.bf16).copy()
    assert not np.array_equal(want, plain), "the gate did not change the output"
    d.out.fill_(float("nan"))
    d.lse.zero_()
    sm = roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows, dim=dim)
    roost_amd.paged_attention_gated(session, p, sm, key=(key, "gated"))
    got = from_dev(d.out, b.bf16)
    assert np.array_equal(got, want), "gated attention differs from attention then SigmoidMul"
    assert np.array_equal(from_dev(d.lse), plain_lse), "the lse of the gated call is not the ungated one"
    # A second gated call on the same plan gives the same bits.
    d.out.fill_(float("nan"))
    roost_amd.paged_attention_gated(session, p, sm, key=(key, "gated"), plan=False)
    assert np.array_equal(from_dev(d.out, b.bf16), want)
    t.cuda.synchronize()


@pytest.mark.parametrize("name,seqs,ps,hnd,causal,window,hd,bf16", GATED_CASES, ids=[c[0] for c in GATED_CASES])
def test_gated_equals_attention_then_sigmoid_mul(session, name, seqs, ps, hnd, causal, window, hd, bf16):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    b = cases.make_paged_batch(rng, [s[1] for s in seqs], [s[0] for s in seqs], page_size=ps, hnd=hnd, d=hd,
                               bf16=bf16)
    _check(session, b, causal, window, key=name)


def test_config5_mixed_step_gated(session):
    """Config 5's attention call (48 decode rows beside two 512-token chunks, the decode rows in the tile pieces' launch) with
    the output gate folded in."""
    rng = np.random.default_rng(5)
    kv = np.concatenate([rng.integers(1024, 16385, size=48), [4608, 4608]])
    n = np.concatenate([np.ones(48, np.int64), [512, 512]])
    b = cases.make_paged_batch(rng, kv, n, std=0.5, pool_factor=1.25)
    _check(session, b, key="config 5")


def test_gated_refusals(session):
    rng = np.random.default_rng(8)
    b = cases.make_paged_batch(rng, [300, 40], [100, 1])
    d = Dev(b)
    p = d.params()
    rows, dim = b.tokens, b.hq * b.d
    gate = _gate(rng, b.q, True)
    other = torch().empty_like(d.out)
    f32_gate = to_dev(np.zeros(b.q.shape, np.float32))

    def status(sm, params=p):
        try:
            roost_amd.paged_attention_gated(session, params, sm, key="refusal")
        except roost_amd.KernelError as e:
            return e.status
        return abi.OK

    ok = roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows, dim=dim)
    assert status(ok) == abi.OK
    assert status(roost_amd.sigmoid_mul_params(other, gate, d.out, rows=rows, dim=dim)) == abi.INVALID_ARGUMENT
    assert status(roost_amd.sigmoid_mul_params(d.out, gate, other, rows=rows, dim=dim)) == abi.INVALID_ARGUMENT
    assert status(roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows - 1, dim=dim)) == abi.INVALID_ARGUMENT
    assert status(roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows, dim=dim // 2)) == abi.INVALID_ARGUMENT
    assert status(roost_amd.sigmoid_mul_params(d.out, f32_gate, d.out, rows=rows, dim=dim)) == abi.INVALID_ARGUMENT
    # The gate may not overlap the output it multiplies.
    assert status(roost_amd.sigmoid_mul_params(d.out, d.out, d.out, rows=rows, dim=dim)) == abi.INVALID_ARGUMENT
    short = roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows, dim=dim)
    short.gate.length = rows * dim - 1
    assert status(short) == abi.INVALID_ARGUMENT
    bad = roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows, dim=dim)
    bad.struct_size = 8
    assert status(bad) == abi.ABI_MISMATCH
    # A refused call leaves the output as it was.
    d.out.fill_(0.0)
    assert status(roost_amd.sigmoid_mul_params(d.out, gate, d.out, rows=rows + 1, dim=dim)) == abi.INVALID_ARGUMENT
    assert not from_dev(d.out, True).any()
