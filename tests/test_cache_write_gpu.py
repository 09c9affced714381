"""CacheWrite on the GPU through the C ABI: bit-exact against the CpuOps oracle (reference
src/Starlings.Roost.Ops/CpuOps.cs:515-569; hand case tests/Starlings.Roost.Ops.Tests/BasicOpsTests.cs:202-232)."""
import numpy as np
import pytest

import cases
import oracle
import roost_amd
from roost_amd import abi
from test_attention_gpu import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _run(session, k, v, kc, vc, slots, *, kv_heads, head_dim, page_size, hnd, bf16):
    dk, dv = to_dev(kc, bf16), to_dev(vc, bf16)
    roost_amd.cache_write(session, to_dev(k, bf16), to_dev(v, bf16), dk, dv, to_dev(slots), kv_heads=kv_heads,
                          head_dim=head_dim, page_size=page_size,
                          kv_layout=abi.LAYOUT_PAGED_HND if hnd else abi.LAYOUT_PAGED_NHD)
    return from_dev(dk, bf16), from_dev(dv, bf16)


@pytest.mark.parametrize("hnd", [False, True])
def test_hand_case(session, hnd):
    # 3 tokens, 2 kv heads, head dim 2, block size 2, 2 blocks; slots [3, -1, 0].
    k = cases.bf16_bits(np.arange(1, 13, dtype=np.float32).reshape(3, 2, 2))
    v = cases.bf16_bits(-np.arange(1, 13, dtype=np.float32).reshape(3, 2, 2))
    kc = np.zeros(16, np.uint16)
    vc = np.zeros(16, np.uint16)
    slots = np.array([3, -1, 0], np.int64)
    gk, gv = _run(session, k, v, kc, vc, slots, kv_heads=2, head_dim=2, page_size=2, hnd=hnd, bf16=True)
    expected = np.zeros(16, np.float32)
    for h in range(2):
        for d in range(2):
            idx = (lambda blk, off: ((blk * 2 + off) * 2 + h) * 2 + d) if not hnd else \
                (lambda blk, off: ((blk * 2 + h) * 2 + off) * 2 + d)
            expected[idx(1, 1)] = h * 2 + d + 1
            expected[idx(0, 0)] = 8 + h * 2 + d + 1
    assert np.array_equal(cases.bf16_values(gk), expected)
    assert np.array_equal(cases.bf16_values(gv), -expected)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("ps", [16, 32])
def test_random_bit_exact_with_skips(session, dtype, hnd, ps):
    rng = np.random.default_rng(ps * 2 + hnd)
    bf16 = dtype == "bf16"
    tokens, hkv, d, pages = 300, 2, 256, 40
    shape = (pages, hkv, ps, d) if hnd else (pages, ps, hkv, d)
    if bf16:
        k = rng.integers(0, 65536, size=(tokens, hkv, d), dtype=np.uint16)
        v = rng.integers(0, 65536, size=(tokens, hkv, d), dtype=np.uint16)
        kc = np.full(shape, 0xABAB, np.uint16)
    else:
        k = rng.standard_normal((tokens, hkv, d), dtype=np.float32)
        v = rng.standard_normal((tokens, hkv, d), dtype=np.float32)
        kc = np.full(shape, np.float32(np.frombuffer(b"\xab\xab\xab\xab", np.float32)[0]))
    vc = kc.copy()
    slots = rng.permutation(pages * ps)[:tokens].astype(np.int64)
    slots[::7] = -1  # negative slots leave the pool untouched
    rk, rv = kc.copy(), vc.copy()
    oracle.cache_write(k, v, rk, rv, slots, tokens=tokens, kv_heads=hkv, head_dim=d, page_size=ps, hnd=hnd, bf16=bf16)
    gk, gv = _run(session, k, v, kc, vc, slots, kv_heads=hkv, head_dim=d, page_size=ps, hnd=hnd, bf16=bf16)
    assert gk.tobytes() == rk.tobytes() and gv.tobytes() == rv.tobytes()


def test_slot_beyond_pool_is_skipped(session):
    rng = np.random.default_rng(3)
    k = rng.integers(0, 65536, size=(4, 2, 64), dtype=np.uint16)
    kc = np.zeros((2, 16, 2, 64), np.uint16)
    slots = np.array([0, 31, 32, 10 ** 9], np.int64)  # 32 and beyond are outside a 2-page pool
    gk, gv = _run(session, k, k, kc, kc.copy(), slots, kv_heads=2, head_dim=64, page_size=16, hnd=False, bf16=True)
    rk = kc.copy()
    oracle.cache_write(k[:2], k[:2], rk, rk.copy(), slots[:2], tokens=2, kv_heads=2, head_dim=64, page_size=16,
                       bf16=True)
    assert gk.tobytes() == rk.tobytes()


def test_unaligned_head_rows_use_the_word_path(session):
    # head_dim 3 (6-byte rows): no 16-byte vectors, still bit-exact.
    rng = np.random.default_rng(8)
    k = rng.integers(0, 65536, size=(5, 2, 3), dtype=np.uint16)
    kc = np.zeros((4, 2, 2, 3), np.uint16)
    slots = np.array([7, 0, -1, 3, 5], np.int64)
    rk = kc.copy()
    oracle.cache_write(k, k, rk, rk.copy(), slots, tokens=5, kv_heads=2, head_dim=3, page_size=2, bf16=True)
    gk, _ = _run(session, k, k, kc, kc.copy(), slots, kv_heads=2, head_dim=3, page_size=2, hnd=False, bf16=True)
    assert gk.tobytes() == rk.tobytes()


def test_rejections(session):
    lib = session.lib
    e = lib.entry(roost_amd.CACHE_WRITE_VARIANT)
    import torch

    k = torch.zeros((2, 2, 64), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((4, 16, 2, 64), dtype=torch.bfloat16, device="cuda")
    s = torch.zeros(2, dtype=torch.int64, device="cuda")
    good = roost_amd.cache_write_params(k, k, kc, kc, s, kv_heads=2, head_dim=64, page_size=16)
    assert session.run_raw(e, good, None) == abi.OK
    p = roost_amd.cache_write_params(k, k, kc, kc, s, kv_heads=2, head_dim=64, page_size=16)
    p.k_scale = 0.5
    assert session.run_raw(e, p, None) == abi.UNSUPPORTED
    p = roost_amd.cache_write_params(k, k, kc, kc, s, kv_heads=2, head_dim=64, page_size=16)
    p.k_cache.dtype = abi.DTYPE_F16
    assert session.run_raw(e, p, None) == abi.UNSUPPORTED
    p = roost_amd.cache_write_params(k, k, kc, kc, s, kv_heads=2, head_dim=64, page_size=16, kv_layout=0)
    assert session.run_raw(e, p, None) == abi.INVALID_ARGUMENT
    p = roost_amd.cache_write_params(k, k, kc, kc, s, kv_heads=2, head_dim=64, page_size=16)
    p.slot_mapping.dtype = abi.DTYPE_I32
    assert session.run_raw(e, p, None) == abi.INVALID_ARGUMENT
    torch.cuda.synchronize()
