"""The allocation-free recurrent GatedDeltaRule entry point (roost_amd_gdn_recurrent_run_noalloc) against the
workspace entry point it mirrors (roost_gdn_recurrent_run), through the C ABI: two routed calls in a row, the second
smaller (the static scratch then holds the first call's tables and records), must give the same outputs and states
bit for bit; a decode-only call needs no scratch; a call beyond the scratch is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

import cases
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev
from test_gdn_gpu import DevGdn

pytestmark = pytest.mark.gpu


def _noalloc(session):
    fn = session.lib.dll.roost_amd_gdn_recurrent_run_noalloc
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    fn.restype = C.c_int32
    return fn


def _both(session, d):
    """(output, pool) from the workspace entry point, then from the allocation-free one, on fresh device copies."""
    ref = DevGdn(d)
    session.launch(session.lib.entry(roost_amd.RECURRENT_VARIANT), ref.params(), key=("noalloc-ref", d.tokens))
    got = DevGdn(d)
    p = got.params()
    status = _noalloc(session)(session.ctx, C.addressof(p), C.c_void_p(session.stream_handle))
    assert status == abi.OK, session.lib.last_error()
    return (from_dev(ref.out, True)[: d.tokens], from_dev(ref.pool)), (from_dev(got.out, True)[: d.tokens],
                                                                      from_dev(got.pool))


@pytest.mark.parametrize("lens_pair", [([600, 1, 17, 40, 1, 300], [100, 3, 16]), ([1] * 8, [1, 1])])
def test_noalloc_matches_workspace_entry_point_twice(session, lens_pair):
    rng = np.random.default_rng(len(lens_pair[0]))
    for lens in lens_pair:  # the second call is smaller and finds the first one's scratch contents
        d = cases.make_gdn(rng, lens, 8, slots=list(range(len(lens))), baseline_style=True)
        (ro, rp), (go, gp) = _both(session, d)
        assert np.array_equal(ro, go), f"outputs differ for lens {lens}"
        assert np.array_equal(rp, gp), f"states differ for lens {lens}"
        want_o, want_pool = cases.oracle_gdn(d)
        cases.assert_close(cases.bf16_values(go), cases.bf16_values(want_o), what=f"noalloc output {lens}")
        for s in range(len(lens)):
            cases.assert_close(gp[s], want_pool[s], max_abs=1.0, max_rel=cases.STATE_REL, what=f"noalloc state {s}")


def test_noalloc_refuses_calls_beyond_its_scratch(session):
    rng = np.random.default_rng(7)
    d = cases.make_gdn(rng, [3000, 3000], 2, slots=[0, 1])
    dev = DevGdn(d)
    before = from_dev(dev.pool)
    p = dev.params()
    assert _noalloc(session)(session.ctx, C.addressof(p), C.c_void_p(session.stream_handle)) == abi.INVALID_ARGUMENT
    assert "scratch" in session.lib.last_error()
    assert np.array_equal(from_dev(dev.pool), before)


@pytest.mark.parametrize("lens", [[1] * 1024, [1] * 1023 + [600]], ids=["decode-1024", "decode-1023-plus-600"])
def test_noalloc_large_batches_bounded_by_the_host_lengths(session, lens):
    """1,024 sequences over 16 value heads: sized from tokens and batch alone these would need more than the static
    scratch holds; the host copy of cu_seqlens bounds the routing to what the batch really chunks (none for a decode
    step, 10 chunks for one 600-token row), so both run, equal to the workspace entry point bit for bit."""
    rng = np.random.default_rng(len(lens))
    d = cases.make_gdn(rng, lens, len(lens), slots=list(range(len(lens))), baseline_style=True)
    (ro, rp), (go, gp) = _both(session, d)
    assert np.array_equal(ro, go)
    assert np.array_equal(rp, gp)
