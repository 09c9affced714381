"""The plan region (roost_amd_plan_region_fill on the host, roost_amd_plan_region_run on the GPU) against the reference's
hand case (tests/Starlings.Roost.Worker.Tests/PlanAndResultTests.cs:25-45) and the restated PlanRegionWriter.Fill
(src/Starlings.Roost.Worker/Eager/PlanRegionWriter.cs:19-64, oracle.plan_region), bit for bit."""
from pathlib import Path

import numpy as np
import pytest

import oracle
import roost_amd
from roost_amd import abi


def _plan(rng, q_lens, kv_lens, block_size=16, pool_factor=1.25):
    """Sequences with disjoint random block lists, laid out token after token."""
    pages = [(kv + block_size - 1) // block_size for kv in kv_lens]
    perm = rng.permutation(int(np.ceil(sum(pages) * pool_factor)) + 1).astype(np.int32)
    seqs, start, used = [], 0, 0
    for n, kv, p in zip(q_lens, kv_lens, pages):
        seqs.append(dict(token_start=start, token_count=int(n), position_offset=int(kv - n), kv_length=int(kv),
                         blocks=perm[used:used + p]))
        start += int(n)
        used += p
    return seqs


def _inputs(seqs, recurrent=True):
    i32 = lambda xs: np.ascontiguousarray(np.asarray(xs, dtype=np.int32))  # noqa: E731
    blocks = [np.asarray(s["blocks"], np.int32) for s in seqs]
    arrays = dict(token_start=i32([s["token_start"] for s in seqs]), token_count=i32([s["token_count"] for s in seqs]),
                  position_offset=i32([s["position_offset"] for s in seqs]),
                  kv_length=i32([s["kv_length"] for s in seqs]),
                  block_indptr=i32(np.concatenate([[0], np.cumsum([b.size for b in blocks])])),
                  blocks=i32(np.concatenate(blocks) if blocks else np.zeros(1, np.int32)))
    if recurrent:
        arrays["recurrent_slot"] = i32([3 * i + 1 for i in range(len(seqs))])
    return arrays


def _outputs(batch, tokens, nblocks, recurrent=True, fill=-7):
    out = dict(q_indptr=np.full(batch + 1, fill, np.int32), cu_seqlens=np.full(batch + 1, fill, np.int32),
               kv_indptr=np.full(batch + 1, fill, np.int32), kv_indices=np.full(max(nblocks, 1), fill, np.int32),
               kv_last_page_len=np.full(max(batch, 1), fill, np.int32), positions=np.full(max(tokens, 1), fill, np.int32),
               slot_mapping=np.full(max(tokens, 1), fill, np.int64))
    if recurrent:
        out["state_slots"] = np.full(max(batch, 1), fill, np.int32)
    return out


def _host_fill(kernels, seqs, block_size=16, tokens=None):
    inp = _inputs(seqs)
    tokens = sum(s["token_count"] for s in seqs) if tokens is None else tokens
    out = _outputs(len(seqs), tokens, int(inp["block_indptr"][-1]))
    roost_amd.plan_region_fill(kernels, batch=len(seqs), tokens=tokens, block_size=block_size, **inp, **out)
    return inp, out


def _check_against_oracle(seqs, out, block_size=16):
    b, tokens = len(seqs), sum(s["token_count"] for s in seqs)
    q_indptr, cu, kv_indptr, kv_indices, last, slots = oracle.plan_region(seqs, block_size)
    assert np.array_equal(out["q_indptr"], q_indptr) and np.array_equal(out["cu_seqlens"], cu)
    assert np.array_equal(out["kv_indptr"], kv_indptr)
    assert np.array_equal(out["kv_indices"][: kv_indices.size], kv_indices)
    assert np.array_equal(out["kv_last_page_len"][:b], last)
    assert np.array_equal(out["slot_mapping"][:tokens], slots)
    want_pos = np.concatenate([np.arange(s["token_count"]) + s["position_offset"] for s in seqs]) if b else []
    assert np.array_equal(out["positions"][:tokens], want_pos)
    if "state_slots" in out and b:
        assert np.array_equal(out["state_slots"][:b], [3 * i + 1 for i in range(b)])


HAND = [dict(token_start=0, token_count=3, position_offset=0, kv_length=3, blocks=[5]),
        dict(token_start=3, token_count=1, position_offset=17, kv_length=18, blocks=[2, 7])]


def test_host_fill_reference_hand_case(kernels):
    _, out = _host_fill(kernels, HAND)
    assert list(out["slot_mapping"]) == [80, 81, 82, 7 * 16 + 1]
    assert list(out["positions"]) == [0, 1, 2, 17]
    assert list(out["q_indptr"]) == [0, 3, 4] and list(out["cu_seqlens"]) == [0, 3, 4]
    assert list(out["kv_indptr"]) == [0, 1, 3] and list(out["kv_indices"]) == [5, 2, 7]
    assert list(out["kv_last_page_len"]) == [3, 2] and list(out["state_slots"]) == [1, 4]


PLANS = [
    ("decode 48 + 2 chunks (worker step)", [1] * 48 + [512, 512], None, 16),
    ("prefill chunks on prefixes", [300, 2048, 256], [300, 8192, 700], 16),
    ("page size 64", [1, 1, 77, 130], [900, 64, 77, 1000], 64),
    ("page size 7", [5, 1, 20], [5, 30, 41], 7),
    ("one sequence on a whole page", [16], [16], 16),
]


def _plan_case(rng, q_lens, kv_lens):
    if kv_lens is None:
        kv_lens = list(rng.integers(1024, 16385, size=sum(1 for q in q_lens if q == 1))) + [4608] * 2
    return q_lens, kv_lens


@pytest.mark.parametrize("name,q_lens,kv_lens,bs", PLANS, ids=[p[0] for p in PLANS])
def test_host_fill_matches_plan_region_writer(kernels, name, q_lens, kv_lens, bs):
    rng = np.random.default_rng(len(name))
    q_lens, kv_lens = _plan_case(rng, q_lens, kv_lens)
    seqs = _plan(rng, q_lens, kv_lens, bs)
    _, out = _host_fill(kernels, seqs, bs)
    _check_against_oracle(seqs, out, bs)


def test_host_fill_empty_batch_and_null_optionals(kernels):
    out = _outputs(0, 0, 0, recurrent=False)
    inp = _inputs([], recurrent=False)
    del out["positions"]
    roost_amd.plan_region_fill(kernels, batch=0, tokens=0, block_size=16, **inp, **out)
    assert out["q_indptr"][0] == 0 and out["cu_seqlens"][0] == 0 and out["kv_indptr"][0] == 0


@pytest.mark.parametrize("change", ["tokens past the end", "position past the blocks", "indptr backwards",
                                   "block size 0", "reserved"])
def test_host_fill_refusals_write_nothing(kernels, change):
    seqs = [dict(s) for s in HAND]
    tokens, bs = 4, 16
    if change == "tokens past the end":
        tokens = 3
    elif change == "position past the blocks":
        seqs[1]["position_offset"] = 32
    inp = _inputs(seqs)
    if change == "indptr backwards":
        inp["block_indptr"] = np.array([0, 2, 1], np.int32)
    if change == "block size 0":
        bs = 0
    out = _outputs(2, 4, 3)
    r = roost_amd.plan_region_struct(batch=2, tokens=tokens, block_size=bs, **inp, **out)
    if change == "reserved":
        r.reserved0 = 1
    import ctypes as C

    assert kernels.dll.roost_amd_plan_region_fill(C.byref(r)) == abi.INVALID_ARGUMENT
    assert kernels.last_error().startswith("plan_region: ")
    assert all((a == -7).all() for a in out.values())


# ---- C2 step plans (roost_amd_plan_region_from_step) ------------------------------------------------------------------

SHM_GOLDEN = Path(__file__).resolve().parent / "golden" / "shm_layout.golden.txt"


def test_step_plan_layouts_match_reference_fixture():
    """The ctypes mirrors the buffers below are built with have the reference's own layout (its fixture, kept as data);
    plan_region.hip pins the same offsets with static_asserts."""
    import ctypes as C

    golden, cur = {}, None
    for line in SHM_GOLDEN.read_text().splitlines():
        if line.startswith("#") or not line.strip():
            continue
        if line.startswith("struct "):
            _, cur, size, _align = line.split()
            golden[cur] = {"size": int(size.split("=")[1]), "fields": []}
            continue
        name, off, size, _type = line.split()
        golden[cur]["fields"].append((name, int(off), int(size)))
    assert set(golden) == set(abi.SHM_STRUCTS)
    for name, st in abi.SHM_STRUCTS.items():
        assert C.sizeof(st) == golden[name]["size"], name
        assert [(f[0], getattr(st, f[0]).offset, getattr(st, f[0]).size) for f in st._fields_] == golden[name]["fields"]


def _step_plan(seqs, *, group_count=3, attention_group=1, sample=None, token_ids=None, seq_stride=80, extra_blocks=2,
               gap=24):
    """A C2 step-plan buffer: header, then the sequence, token-id, position, group-block and block-id tables (each
    after `gap` bytes of 0xEE filler, the sequence table at `seq_stride` bytes per entry). Every sequence lists
    `extra_blocks` blocks more than it needs in the attention group, and decoy lists in the other groups."""
    import ctypes as C

    b = len(seqs)
    tokens = sum(s["token_count"] for s in seqs)
    token_ids = np.arange(tokens, dtype=np.int32) * 7 + 3 if token_ids is None else token_ids
    sample = [i % 2 == 0 for i in range(b)] if sample is None else sample
    block_ids, groups = [], []
    for i, s in enumerate(seqs):
        for g in range(group_count):
            if g == attention_group:
                lst = list(s["blocks"]) + [900000 + i * 10 + j for j in range(extra_blocks)]
            else:
                lst = [800000 + i * 10 + g]
            groups.append((len(block_ids), len(lst)))
            block_ids += lst
    parts, at = [], C.sizeof(abi.StepPlanHeader)

    def place(raw):
        nonlocal at
        at += gap
        parts.append((at, raw))
        off = at
        at += len(raw)
        return off

    seq_raw = bytearray()
    for i, s in enumerate(seqs):
        ps = abi.PlanSequence(sequence_handle=1000 + i, token_start=s["token_start"], token_count=s["token_count"],
                              position_offset=s["position_offset"], group_blocks_start=i * group_count,
                              recurrent_slot=5 * i + 2, lora_slot=-1, grammar_slot=-1, embedding_slot=-1,
                              flags=abi.SEQ_FLAG_SAMPLE if sample[i] else 0, head_row=-1, encoder_output=-1)
        seq_raw += bytes(ps) + b"\xEE" * (seq_stride - C.sizeof(ps))
    positions = (np.concatenate([np.arange(s["token_count"]) + s["position_offset"] for s in seqs]).astype(np.int32)
                 if b else np.zeros(0, np.int32))
    gb_raw = b"".join(bytes(abi.PlanGroupBlocks(a, n)) for a, n in groups)
    h = abi.StepPlanHeader(magic=abi.SHM_MAGIC_PLAN, layout_version=abi.SHM_LAYOUT_VERSION,
                           header_size=C.sizeof(abi.StepPlanHeader), step_id=11, sequence_count=b, token_count=tokens,
                           group_count=group_count)
    h.sequences = abi.TableRef(place(bytes(seq_raw)), b, seq_stride)
    h.token_ids = abi.TableRef(place(np.asarray(token_ids, np.int32).tobytes()), tokens, 4)
    h.positions = abi.TableRef(place(positions.tobytes()), tokens, 4)
    h.group_blocks = abi.TableRef(place(gb_raw), b * group_count, 8)
    h.block_ids = abi.TableRef(place(np.asarray(block_ids, np.int32).tobytes()), len(block_ids), 4)
    h.total_bytes = at
    buf = bytearray(b"\xEE" * at)
    buf[: C.sizeof(h)] = bytes(h)
    for off, raw in parts:
        buf[off:off + len(raw)] = raw
    return np.frombuffer(bytes(buf), dtype=np.uint8).copy(), token_ids, sample


def _from_step(kernels, buf, seqs, bs, **kw):
    tokens = sum(s["token_count"] for s in seqs)
    nblocks = sum(len(s["blocks"]) for s in seqs)
    pool = 1 + max((b for s in seqs for b in s["blocks"]), default=0)
    args = dict(attention_group=1, block_size=bs, attention_blocks=pool, max_batch=len(seqs), max_tokens=tokens,
                max_blocks=nblocks)
    args.update(kw)
    return roost_amd.plan_region_from_step(kernels, buf, **args)


@pytest.mark.parametrize("name,q_lens,kv_lens,bs", PLANS, ids=[p[0] for p in PLANS])
def test_step_plan_matches_plan_region_writer(kernels, name, q_lens, kv_lens, bs):
    rng = np.random.default_rng(len(name) + 100)
    q_lens, kv_lens = _plan_case(rng, q_lens, kv_lens)
    seqs = _plan(rng, q_lens, kv_lens, bs)
    buf, ids, sample = _step_plan(seqs, seq_stride=96 if bs == 7 else 80)
    out = _from_step(kernels, buf, seqs, bs)
    q_indptr, cu, kv_indptr, kv_indices, last, slots = oracle.plan_region(seqs, bs)
    assert np.array_equal(out["q_indptr"], q_indptr) and np.array_equal(out["cu_seqlens"], cu)
    assert np.array_equal(out["kv_indptr"], kv_indptr) and np.array_equal(out["kv_indices"], kv_indices)
    assert np.array_equal(out["kv_last_page_len"], last) and np.array_equal(out["slot_mapping"], slots)
    assert np.array_equal(out["positions"], np.concatenate([np.arange(s["token_count"]) + s["position_offset"]
                                                            for s in seqs]))
    assert np.array_equal(out["ids"], ids)
    assert np.array_equal(out["state_slots"], [5 * i + 2 for i in range(len(seqs))])
    want_rows = [s["token_start"] + s["token_count"] - 1 for s, smp in zip(seqs, sample) if smp]
    assert list(out["rows"]) == want_rows


def test_step_plan_reference_hand_case(kernels):
    """PlanAndResultTests.cs:25-45's plan: a 3-token prefill from position 0 and a decode at position 17."""
    buf, _, _ = _step_plan(HAND, sample=[False, True], token_ids=np.array([11, 12, 13, 14], np.int32))
    out = _from_step(kernels, buf, HAND, 16)
    assert list(out["slot_mapping"]) == [80, 81, 82, 7 * 16 + 1] and list(out["positions"]) == [0, 1, 2, 17]
    assert list(out["kv_indptr"]) == [0, 1, 3] and list(out["kv_indices"]) == [5, 2, 7]
    assert list(out["kv_last_page_len"]) == [3, 2] and list(out["ids"]) == [11, 12, 13, 14] and list(out["rows"]) == [3]


def test_step_plan_empty(kernels):
    buf, _, _ = _step_plan([])
    out = roost_amd.plan_region_from_step(kernels, buf, attention_group=1, block_size=16, attention_blocks=1,
                                          max_batch=0, max_tokens=0, max_blocks=0)
    assert list(out["q_indptr"]) == [0] and list(out["kv_indptr"]) == [0] and out["rows"].size == 0


@pytest.mark.parametrize("change", ["magic", "short buffer", "table past the end", "tokens not contiguous",
                                   "positions skip", "too few blocks", "group_blocks_start", "attention group",
                                   "outputs too small", "token count", "block id past the pool",
                                   "negative block id", "no pool size"])
def test_step_plan_refusals(kernels, change):
    import ctypes as C

    seqs = [dict(s, blocks=list(s["blocks"])) for s in HAND]
    kw = dict(extra_blocks=0)
    call = {}
    buf, _, _ = _step_plan(seqs, **kw)
    h = abi.StepPlanHeader.from_buffer_copy(bytes(buf[:C.sizeof(abi.StepPlanHeader)]))
    seq_at = lambda i: int(h.sequences.offset) + i * int(h.sequences.stride)  # noqa: E731
    if change == "magic":
        buf[0] ^= 1
    elif change == "short buffer":
        buf = buf[:-1]
    elif change == "table past the end":
        h.block_ids.offset = h.total_bytes - 4
        buf[:C.sizeof(h)] = np.frombuffer(bytes(h), np.uint8)
    elif change == "tokens not contiguous":
        buf[seq_at(1) + 8] += 1  # token_start 3 -> 4
    elif change == "positions skip":
        pos_at = int(h.positions.offset) + 4
        buf[pos_at] += 1
    elif change == "too few blocks":
        seqs[1]["position_offset"] = 40  # 41 keys need 3 blocks of 16; 2 are listed
        buf, _, _ = _step_plan(seqs, **kw)
    elif change == "group_blocks_start":
        buf[seq_at(1) + 20] += 1
    elif change == "attention group":
        call["attention_group"] = 3
    elif change == "outputs too small":
        call["max_tokens"] = 3
    elif change == "block id past the pool":
        call["attention_blocks"] = 7  # the hand case lists block 7
    elif change == "negative block id":
        seqs[1]["blocks"][0] = -1
        buf, _, _ = _step_plan(seqs, **kw)
        call["attention_blocks"] = 8
    elif change == "no pool size":
        call["attention_blocks"] = 0
    elif change == "token count":
        h.token_count += 1
        buf[:C.sizeof(h)] = np.frombuffer(bytes(h), np.uint8)
    with pytest.raises(roost_amd.KernelError) as err:
        _from_step(kernels, buf, HAND, 16, **call)
    assert err.value.status == abi.INVALID_ARGUMENT and "plan_region: " in str(err.value)


# ---- device path -------------------------------------------------------------------------------------------------------

def _device_run(session, seqs, bs, tokens=None, fill=-7):
    import torch

    inp = {k: torch.from_numpy(v).cuda() for k, v in _inputs(seqs).items()}
    tokens = sum(s["token_count"] for s in seqs) if tokens is None else tokens
    nb = int(inp["block_indptr"][-1].item()) if seqs else 0
    out = {k: torch.from_numpy(v).cuda() for k, v in _outputs(len(seqs), tokens, nb, fill=fill).items()}
    roost_amd.plan_region_run(session, batch=len(seqs), tokens=tokens, block_size=bs, **inp, **out)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.gpu
@pytest.mark.parametrize("name,q_lens,kv_lens,bs", PLANS, ids=[p[0] for p in PLANS])
def test_device_run_matches_host_fill(session, kernels, name, q_lens, kv_lens, bs):
    rng = np.random.default_rng(len(name))
    q_lens, kv_lens = _plan_case(rng, q_lens, kv_lens)
    seqs = _plan(rng, q_lens, kv_lens, bs)
    got = _device_run(session, seqs, bs)
    _check_against_oracle(seqs, got, bs)
    _, want = _host_fill(kernels, seqs, bs)
    for k in want:
        assert np.array_equal(got[k], want[k]), k


@pytest.mark.gpu
def test_device_run_hand_case_empty_batch_and_unmapped_positions(session):
    got = _device_run(session, HAND, 16)
    assert list(got["slot_mapping"]) == [80, 81, 82, 113] and list(got["kv_last_page_len"]) == [3, 2]
    empty = _device_run(session, [], 16)
    assert empty["q_indptr"][0] == 0 and empty["kv_indptr"][0] == 0 and (empty["slot_mapping"] == -7).all()
    # Device data is not validated on the host: a position past the blocks gets slot -1, a token past `tokens` is
    # skipped.
    seqs = [dict(s) for s in HAND]
    seqs[1]["position_offset"] = 32
    got = _device_run(session, seqs, 16, tokens=3)
    assert list(got["slot_mapping"][:3]) == [80, 81, 82] and got["slot_mapping"].size == 3
    got = _device_run(session, seqs, 16)
    assert got["slot_mapping"][3] == -1
