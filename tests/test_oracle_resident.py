"""Pins the resident-round oracle (oracle/resident.py).

- The reference's stateful known answer (tests/operators/lifetch/support/correctness.py:
  170-228): batch 2, history 12288, resident 4096, 32 heads, fixed Index keys with three
  2048-position feature blocks; rounds A, A, B+C, A read 2048, 0, 4096, 2048 rows per
  request, B/C evict A and every selected token ends up hot. Run with the oracle's real
  LI (oracle.indexer.li_keys), TopK and SlotLRU between rounds.
- The reference's acceptance invariants after every round (tests/operators/lifetch/support/
  execution.py:2109-2198): slot output inside the hot cache, the hot cache at each
  selected slot holds that token's KV, logical output = pre-update logical ids, and every
  valid hot slot holds the KV of the logical id its Index row carries.
- The boundary rule "duplicate Q3/Q4 must issue no new repair" (correctness.py:160-163).
- Hand known answers for the allocation order, change records and the chunked
  permutation, and brute-force properties of apply_changes.
"""
import numpy as np
import pytest

from oracle import cache as lru_ref
from oracle import indexer as li_ref
from oracle import resident as ref

TOPK = ref.TOPK


def make_state(owners_history, resident, row_bytes=656, rng=None, hot_valid=1):
    history = owners_history
    keys = np.zeros((history, 128), np.uint8)
    scales = np.ones(history, np.float32)
    addresses = np.arange(history, dtype=np.int64) * row_bytes
    logical = np.arange(history, dtype=np.int64)
    pool = li_ref.identity_rows(np.arange(history), row_bytes)
    hot_cache = pool[:resident].copy()
    valid = np.full(resident, hot_valid, np.int64)
    return dict(keys=keys, scales=scales, addresses=addresses, logical=logical, pool=pool.reshape(-1),
                hot_cache=hot_cache, hot_valid=valid, history=history, resident=resident)


def check_invariants(st, selected, logical_before, lout, sout):
    """execution.py:2109-2198 for one request."""
    resident = st["resident"]
    live = selected >= 0
    assert np.array_equal(lout[live], logical_before[selected[live]])
    assert (lout[~live] == -1).all() and (sout[~live] == -1).all()
    assert ((sout[live] >= 0) & (sout[live] < resident)).all()
    pool = st["pool"].reshape(-1, st["hot_cache"].shape[1])
    for s, token in zip(sout[live], lout[live]):
        assert np.array_equal(st["hot_cache"][s], pool[token])
    for s in np.nonzero(st["hot_valid"])[0]:
        assert np.array_equal(st["hot_cache"][s], pool[st["logical"][s]]), s
    # Distinct positions of one row occupy distinct slots.
    for q in range(selected.shape[0]):
        m = selected[q] >= 0
        assert len(set(sout[q][m].tolist())) == int(m.sum())


def run_round(st, selected, lru, used=0):
    reserved = ref.reserved_from_candidates(lru, st["resident"])
    before = st["logical"].copy()
    lout, sout, res, err = ref.resident_round(selected, st["history"], st["resident"], st["keys"], st["scales"],
                                              st["addresses"], st["logical"], st["hot_valid"], reserved, lru,
                                              st["hot_cache"], st["pool"], used)
    assert err == 0
    check_invariants(st, selected, before, lout, sout)
    return lout, sout, res


def test_stateful_known_answer_a_a_bc_a():
    """correctness.py:170-228: reads per request 2048, 0, 4096, 2048."""
    history, resident, heads = 12288, 4096, 32
    st = make_state(history, resident)
    fp8_one = 0x38
    for feature, begin in enumerate((4096, 6144, 8192)):
        st["keys"][begin:begin + 2048, feature] = fp8_one
    policy = lru_ref.SlotLRU()
    policy.resize(resident, resident)
    ends = np.arange(history - 3, history + 1)
    reads = []
    for number in range(1, 5):
        features = (1, 2, 1, 2) if number == 3 else (0, 0, 0, 0)
        key_vals = li_ref.fp8_e4m3_decode(st["keys"])
        selected = np.full((4, TOPK), -1, np.int64)
        for q, feature in enumerate(features):
            query = np.zeros((heads, 128), np.float32)
            query[:, feature] = 1.0
            k = li_ref.li_keys(query, key_vals, np.ones(heads, np.float32))
            valid = min(history, int(ends[q]))
            selected[q] = li_ref.topk_reference(k, valid)
        lru = policy.slots.astype(np.int64).copy()
        lout, sout, res = run_round(st, selected, lru)
        reads.append(int(res["added"].sum()))
        policy.commit(sout[sout >= 0])
        # Selected tokens are resident afterwards; B/C evict A in round 3.
        hot_tokens = set(st["logical"][:resident][st["hot_valid"] != 0].tolist())
        expected = set(range(6144, 10240)) if number == 3 else set(range(4096, 6144))
        assert expected <= hot_tokens, number
        if number == 3:
            assert not hot_tokens & set(range(4096, 6144))
            assert list(res["added"]) == [2048, 2048, 0, 0]
    assert reads == [2048, 0, 4096, 2048]


def test_duplicate_q3_q4_issue_no_new_repair_and_cross_query_dedup():
    """correctness.py:160-163 and the same-position shortcut (resolver_staged_dma2.h:133-136)."""
    st = make_state(16384, 8192)
    rng = np.random.default_rng(3)
    a = rng.permutation(np.arange(8192, 16384))[:TOPK]
    b = rng.permutation(np.arange(8192, 16384))[:TOPK]
    selected = np.stack([a, b, a, b])
    lru = np.arange(2048)
    lout, sout, res = run_round(st, selected, lru)
    shared = len(set(a.tolist()) & set(b.tolist()))
    assert list(res["added"]) == [2048, 2048 - shared, 0, 0]
    assert np.array_equal(sout[2], sout[0]) and np.array_equal(sout[3], sout[1])
    # Rank order: row 0's misses take the candidates in ordinal order, by index; row 1's
    # new misses take the lowest free hot slots (candidates exhausted).
    assert np.array_equal(sout[0], lru)
    assert np.array_equal(res["slots"][2048:], np.arange(2048, 2048 + 2048 - shared))


def test_known_answer_hits_miss_order_and_records():
    st = make_state(4096, 2048)
    st["hot_valid"][5] = 0                       # position 5: hot but invalid -> miss
    lru = np.concatenate([np.arange(100, 2048), np.arange(0, 100)])  # 7, 10 are candidates
    selected = np.full((1, TOPK), -1, np.int64)
    selected[0, :6] = [3000, 7, 2050, 5, 11, 3000 + 1]
    reserved = ref.reserved_from_candidates(lru, 2048)
    res = ref.resolve(selected, 4096, 2048, st["hot_valid"], reserved, lru)
    # 7 is a candidate (reserved) -> miss; 5 invalid -> miss; 11 reserved too -> miss.
    assert res["loc"][0, :6].tolist() == [100, 101, 102, 103, 104, 105]
    assert res["tokens"].tolist() == [3000, 7, 2050, 5, 11, 3001]
    # Records: reserved ordinal of the slot when it is a candidate (all are here).
    for r, s in enumerate(range(100, 106)):
        assert res["change_slots"][s - 100] == s and res["changes"][s - 100] == res["tokens"][r]
    assert np.array_equal(res["change_slots"][6:2048], lru[6:2048])
    # A valid hot position that is not a candidate is a hit, keeps its slot and needs no
    # Fetch; the misses around it still take candidates in order.
    st = make_state(8192, 4096)
    lru = np.arange(2048, 4096)
    selected = np.full((1, TOPK), -1, np.int64)
    selected[0, :3] = [5000, 100, 6000]
    res = ref.resolve(selected, 8192, 4096, st["hot_valid"], ref.reserved_from_candidates(lru, 4096), lru)
    assert res["loc"][0, :3].tolist() == [2048, 100, 2049]
    assert res["tokens"].tolist() == [5000, 6000] and list(res["added"]) == [2]


def test_fallback_takes_lowest_free_hot_slots():
    """resolver_staged_dma2.h:189-217: candidates exhausted -> ascending free hot slots,
    every known slot of every row protected."""
    resident = 4096
    st = make_state(16384, resident)
    lru = np.arange(2048, 4096)  # only the upper half are candidates
    rng = np.random.default_rng(5)
    hit_pos = np.arange(0, 40)   # hits on 0..39 (valid, not candidates)
    cold = rng.permutation(np.arange(resident, 16384))
    selected = np.stack([np.concatenate([hit_pos, cold[:2008]]), cold[2008:2008 + TOPK]])
    reserved = ref.reserved_from_candidates(lru, resident)
    res = ref.resolve(selected, 16384, resident, st["hot_valid"], reserved, lru)
    assert res["error"] == 0
    assert list(res["added"]) == [2008, 2048]
    # Row 0 takes candidates 2048..4055; row 1 takes the last 40 candidates, then the
    # free hot slots from 40 upwards (0..39 hold row 0's hits).
    assert np.array_equal(res["slots"][:2008], np.arange(2048, 4056))
    assert np.array_equal(res["slots"][2008:2048], np.arange(4056, 4096))
    assert np.array_equal(res["slots"][2048:], np.arange(40, 40 + 2008))


def test_candidate_outside_hot_range_fails_the_request():
    st = make_state(4096, 2048)
    lru = np.arange(2048)
    lru[7] = 5000
    selected = np.full((1, TOPK), -1, np.int64)
    selected[0, 0] = 3000
    res = ref.resolve(selected, 4096, 2048, st["hot_valid"], ref.reserved_from_candidates(lru, 2048), lru)
    assert res["error"] & ref.ERR_CANDIDATE


def test_duplicate_candidates_fail_the_request_and_clear_residency():
    """A hot slot named by two candidates fails the request before anything moves: both
    outputs -1, the owner's hot_valid cleared (index_cache_update.h:5-21), every other table
    unchanged."""
    st = make_state(8192, 4096)
    lru = np.arange(2048, 4096)
    lru[9] = lru[1500]
    selected = np.full((2, TOPK), -1, np.int64)
    selected[:, :3] = [[10, 5000, 6000], [11, 5000, 7000]]
    before = {k: v.copy() for k, v in st.items() if isinstance(v, np.ndarray)}
    lout, sout, res, err = ref.resident_round(
        selected, st["history"], st["resident"], st["keys"], st["scales"], st["addresses"], st["logical"],
        st["hot_valid"], ref.reserved_from_candidates(lru, 4096), lru, st["hot_cache"], st["pool"])
    assert err == ref.ERR_CANDIDATE
    assert (lout == -1).all() and (sout == -1).all()
    assert not st["hot_valid"].any()
    for k, v in before.items():
        if k != "hot_valid":
            assert np.array_equal(st[k], v), k
    # Padding (-1) candidates may repeat.
    lru2 = np.full(2048, -1)
    lru2[:100] = np.arange(100)
    res = ref.resolve(np.full((1, TOPK), -1, np.int64), 8192, 4096, np.ones(4096), 
                      ref.reserved_from_candidates(lru2, 4096), lru2)
    assert res["error"] == 0


def test_source_outside_the_pool_fails_before_the_fetch():
    """A miss whose KV address lies outside the host pool (or is not 16-byte aligned) fails
    its request before anything is fetched: -1 outputs, residency cleared, hot cache and
    Index untouched."""
    for bad in (None, 5):
        st = make_state(8192, 4096)
        st["addresses"][5000] = st["pool"].size if bad is None else st["addresses"][5000] + bad
        hot_before = st["hot_cache"].copy()
        logical_before = st["logical"].copy()
        lru = np.arange(2048)
        selected = np.full((1, TOPK), -1, np.int64)
        selected[0, :3] = [5000, 6000, 7000]
        lout, sout, res, err = ref.resident_round(
            selected, st["history"], st["resident"], st["keys"], st["scales"], st["addresses"], st["logical"],
            st["hot_valid"], ref.reserved_from_candidates(lru, 4096), lru, st["hot_cache"], st["pool"])
        assert err == ref.ERR_SOURCE
        assert (lout == -1).all() and (sout == -1).all() and not st["hot_valid"].any()
        assert np.array_equal(st["hot_cache"], hot_before) and np.array_equal(st["logical"], logical_before)


def test_rejected_later_chunk_keeps_a_consistent_permutation():
    """A chunk rejected after earlier chunks were applied: the earlier chunks stay applied
    and every table is still one permutation of the original rows (keys, scales, addresses
    and logical ids moving together). The mistake is planted in the oracle's input: the
    second chunk repeats a destination."""
    history, resident = 4096, 2048
    rng = np.random.default_rng(4)
    keys = rng.integers(0, 256, (history, 128), dtype=np.uint8)
    scales = rng.random(history).astype(np.float32)
    addresses = np.arange(history, dtype=np.int64) * 656
    logical = np.arange(history, dtype=np.int64)
    valid = np.ones(resident, np.int64)
    k0, s0, a0 = keys.copy(), scales.copy(), addresses.copy()
    origs = rng.choice(np.arange(resident, history), ref.CHUNK + 10, replace=False)
    dsts = rng.choice(resident, ref.CHUNK + 10, replace=False)
    dsts[ref.CHUNK + 3] = dsts[ref.CHUNK + 1]  # duplicate destination in chunk 2
    batch = list(zip(origs.tolist(), dsts.tolist()))
    err = ref.apply_changes([batch], history, resident, keys, scales, addresses, logical, valid)
    assert err == ref.ERR_UPDATE
    assert np.array_equal(np.sort(logical), np.arange(history))
    assert np.array_equal(keys, k0[logical]) and np.array_equal(scales, s0[logical])
    assert np.array_equal(addresses, a0[logical])
    # Chunk 1 applied: each of its tokens sits at its destination.
    for o, d in batch[:ref.CHUNK]:
        assert logical[d] == o
    # Chunk 2 not applied: its sources still hold their own rows.
    for o, d in batch[ref.CHUNK:]:
        assert logical[o] == o


def test_failure_after_the_fetch_clears_residency(monkeypatch):
    """resident_round when the Index update rejects its changes after the Fetch: the owner
    loses all residency and the outputs stay as published. The failure is planted in the
    oracle by a resolve result whose later miss repeats a slot."""
    st = make_state(8192, 4096)
    lru = np.arange(2048, 4096)
    selected = np.full((1, TOPK), -1, np.int64)
    selected[0, :600] = np.arange(5000, 5600)
    real = ref.resolve

    def broken(*args, **kw):
        res = real(*args, **kw)
        res["slots"] = res["slots"].copy()
        res["slots"][599] = res["slots"][550]
        return res

    monkeypatch.setattr(ref, "resolve", broken)
    lout, sout, res, err = ref.resident_round(
        selected, st["history"], st["resident"], st["keys"], st["scales"], st["addresses"], st["logical"],
        st["hot_valid"], ref.reserved_from_candidates(lru, 4096), lru, st["hot_cache"], st["pool"])
    assert err == ref.ERR_UPDATE
    assert not st["hot_valid"].any()
    assert np.array_equal(lout[0, :600], np.arange(5000, 5600))
    # The first 512-change chunk was applied.
    assert np.array_equal(st["logical"][2048:2048 + 512], np.arange(5000, 5512))


def test_apply_changes_chunk_closure_known_answer():
    """shadow_exchange_parallel.h:28-78 on a hand case: 2 changes, one destination is also
    a source; the displaced row fills the freed position, which loses residency."""
    history, resident = 256, 128
    keys = np.arange(history, dtype=np.uint8)[:, None].repeat(128, 1)
    scales = np.arange(history, dtype=np.float32)
    addresses = np.arange(history, dtype=np.int64) * 10
    logical = np.arange(history, dtype=np.int64) + 1000
    valid = np.ones(resident, np.int64)
    # Row at 200 -> slot 5; row at 5 -> slot 9: slot 9's row is displaced into 200's place.
    err = ref.apply_changes([[(200, 5), (5, 9)]], history, resident, keys, scales, addresses, logical, valid)
    assert err == 0
    assert keys[5, 0] == 200 and keys[9, 0] == 5 and keys[200, 0] == 9
    assert logical[5] == 1200 and logical[9] == 1005 and logical[200] == 1009
    assert addresses[200] == 90 and scales[200] == 9
    assert valid.sum() == resident  # freed position 200 is cold
    # Second batch refers to original rows: original row 9 (now at 200) -> slot 1; the
    # displaced row of slot 1 fills 200 and position 200 is cold, so nothing is invalidated.
    err = ref.apply_changes([[(200, 5), (5, 9)], [(9, 1)]], history, resident, *[
        np.arange(history, dtype=np.uint8)[:, None].repeat(128, 1), np.arange(history, dtype=np.float32),
        np.arange(history, dtype=np.int64) * 10, np.arange(history, dtype=np.int64) + 1000, valid])
    assert err == 0


def test_apply_changes_is_a_permutation_brute_force():
    rng = np.random.default_rng(11)
    history, resident = 4096, 1024
    for trial in range(20):
        keys = rng.integers(0, 256, (history, 128), dtype=np.uint8)
        keys[:, :8] = np.arange(history, dtype=np.uint64).view(np.uint8).reshape(history, 8)
        before = keys.copy()
        scales = np.arange(history, dtype=np.float32)
        addresses = np.arange(history, dtype=np.int64)
        logical = np.arange(history, dtype=np.int64)
        valid = np.ones(resident, np.int64)
        n = int(rng.integers(1, 1000))
        origs = rng.choice(history, n, replace=False)
        dsts = rng.choice(resident, n, replace=False)
        splits = sorted(rng.choice(np.arange(1, n), min(2, n - 1), replace=False).tolist()) if n > 2 else []
        bounds = [0] + splits + [n]
        batches = [list(zip(origs[a:b].tolist(), dsts[a:b].tolist())) for a, b in zip(bounds[:-1], bounds[1:])]
        assert ref.apply_changes(batches, history, resident, keys, scales, addresses, logical, valid) == 0
        # A permutation of rows, with every moved row at its destination, metadata in step.
        assert sorted(logical.tolist()) == list(range(history))
        assert np.array_equal(keys, before[logical])
        assert np.array_equal(scales, logical.astype(np.float32)) and np.array_equal(addresses, logical)
        for o, d in zip(origs, dsts):
            assert logical[d] == o
        # Positions no change touched keep their rows.
        touched = set(origs.tolist()) | set(dsts.tolist())
        for p in rng.choice(history, 64):
            if p not in touched:
                assert logical[p] == p
        # Only positions a change touched can lose residency (freed sources).
        for p in np.nonzero(valid == 0)[0]:
            assert p in touched
        # A single chunk: exactly the freed hot sources (not destinations) lose residency.
        if len(batches) == 1 and n <= ref.CHUNK:
            freed = set(origs.tolist()) - set(dsts.tolist())
            assert set(np.nonzero(valid == 0)[0].tolist()) == {p for p in freed if p < resident}


def test_apply_changes_rejects_non_permutations():
    history, resident = 512, 256
    z = lambda: (np.zeros((history, 128), np.uint8), np.zeros(history, np.float32), np.zeros(history, np.int64),
                 np.zeros(history, np.int64), np.ones(resident, np.int64))
    assert ref.apply_changes([[(300, 5), (301, 5)]], history, resident, *z()) == ref.ERR_UPDATE
    assert ref.apply_changes([[(300, 5), (300, 6)]], history, resident, *z()) == ref.ERR_UPDATE
    assert ref.apply_changes([[(300, resident)]], history, resident, *z()) == ref.ERR_UPDATE


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_multi_round_invariants(seed):
    """Four rounds of random Q=1..4 selections with ~70 % hot picks, the oracle SlotLRU
    supplying candidates; the reference's acceptance invariants hold after every round."""
    rng = np.random.default_rng(seed)
    history, resident = 16384, 4096
    st = make_state(history, resident)
    st["hot_valid"][rng.random(resident) < 0.1] = 0
    policy = lru_ref.SlotLRU()
    policy.resize(resident, resident)
    q_rows = int(rng.integers(1, 5))
    for rnd in range(4):
        # The rows of one request (decode + MTP) share most of their selection.
        n = int(rng.integers(1500, TOPK + 1))
        hot = rng.choice(resident, int(n * 0.7), replace=False)
        cold = rng.choice(np.arange(resident, history), n - len(hot), replace=False)
        base = rng.permutation(np.concatenate([hot, cold]))
        selected = np.full((q_rows, TOPK), -1, np.int64)
        for q in range(q_rows):
            row = base.copy()
            swap = rng.random(n) < 0.1
            row[swap] = rng.choice(np.setdiff1d(np.arange(history), base), int(swap.sum()), replace=False)
            selected[q, :n] = rng.permutation(row)
        lout, sout, res = run_round(st, selected, policy.slots.astype(np.int64).copy())
        policy.commit(sout[sout >= 0])


def test_prefix_classify_closed_forms():
    """Threshold = the resident selection's kth key (the smallest selected key, the TopK's
    own cut), hits = strict comparisons against it (ClassifyScore uses CMPMODE::GT)."""
    rng = np.random.default_rng(4)
    resident, valid, key_stride = 4096, 10000, 10240
    keys = rng.integers(0x8000, 0x8400, key_stride).astype(np.uint16)
    lru = rng.permutation(resident)[:2048]
    lru[:3] = [resident + 5, 9999, -1]  # outside the prefix: never hits
    sel, thr, victim, cold = ref.prefix_classify(keys, valid, resident, lru, (key_stride - resident + 31) // 32)
    assert np.array_equal(sel, li_ref.topk_reference(keys, resident))
    assert thr == np.sort(keys[:resident])[::-1][2047]
    bits = np.unpackbits(victim.view(np.uint8), bitorder="little")
    want = np.array([0 <= s < resident and keys[s] > thr for s in lru])
    assert np.array_equal(bits.astype(bool), want)
    cbits = np.unpackbits(cold.view(np.uint8), bitorder="little")[:key_stride - resident].astype(bool)
    wantc = (keys[resident:] > thr) & (np.arange(resident, key_stride) < valid)
    assert np.array_equal(cbits, wantc)
    # A short prefix selects everything below it and has threshold 0.
    sel, thr, _, _ = ref.prefix_classify(keys, 1000, resident, lru, 200)
    assert thr == 0 and np.array_equal(sel[:1000], np.arange(1000)) and (sel[1000:] == -1).all()


# ----------------------------------------------------------------------------
# ABC tail bounds
# ----------------------------------------------------------------------------
def _tail_mapping_literal(history, resident, ring, begin, end):
    """The reference's round-start tail mapping written out as its loop
    (prefetch.h:25-43: mapping[begin + i] = resident + kSlots + (begin + i) % ring for
    i < ring while begin + i < end and < history) followed by ResolvePhysicalSlot
    (cache_metadata.h:102-106, no LRU ordinal range hit: slot - kSlots)."""
    k_slots = 8192
    mapping = np.full(history, 0xFFFFFFFF, np.int64)
    for i in range(ring):
        t = begin + i
        if t < end and t < history:
            mapping[t] = resident + k_slots + t % ring
    resolved = np.where((mapping >= resident + k_slots) & (mapping < 0x80000000), mapping - k_slots, -1)
    return resolved


def test_tail_slot_equals_the_literal_mapping_loop():
    history, resident, ring = 9000, 2048, 384
    for begin, end in [(0, 0), (5000, 5100), (5000, 5384), (5000, 6000), (100, 900), (8800, 9000), (0, 9000)]:
        want = _tail_mapping_literal(history, resident, ring, begin, end)
        for t in range(history):
            in_tail, slot = ref.tail_slot(t, (begin, end, ring))
            assert in_tail == (begin <= t < end)
            got = -1 if slot is None else resident + slot
            assert got == want[t], (begin, end, t)


def test_tail_positions_known_answer():
    """Hand case: hot, valid positions inside the tail are not hits; the first `ring`
    tail positions resolve to ring slots without a Fetch; later ones are misses."""
    history, resident, ring = 8192, 4096, 384
    hot_valid = np.ones(resident, np.int32)
    lru = np.arange(2048, 4096, dtype=np.int64)  # candidates: the upper half of the hot slots
    reserved = ref.reserved_from_candidates(lru, resident)
    sel = np.full((1, TOPK), -1, np.int64)
    # 100 and 483: tail and mapped (100 + 384 = 484); 484: tail, unmapped -> miss; 50: hot
    # hit; 5000: cold -> miss.
    sel[0, :5] = [100, 483, 484, 50, 5000]
    res = ref.resolve(sel, history, resident, hot_valid, reserved, lru, tail=(100, 600, ring))
    assert res["error"] == 0
    assert res["loc"][0, 0] == resident + 100 % ring  # 4196
    assert res["loc"][0, 1] == resident + 483 % ring  # 4195
    assert res["loc"][0, 3] == 50
    assert res["tokens"].tolist() == [484, 5000]
    assert res["slots"].tolist() == [2048, 2049]  # the first free candidates, in ordinal order
    # Without the tail, 100 and 483 are hot hits.
    plain = ref.resolve(sel, history, resident, hot_valid, reserved, lru)
    assert plain["loc"][0, 0] == 100 and plain["loc"][0, 1] == 483 and plain["loc"][0, 2] == 484
    assert plain["tokens"].tolist() == [5000]
    # Tail bounds outside 0 <= begin <= end <= history fail the request.
    bad = ref.resolve(sel, history, resident, hot_valid, reserved, lru, tail=(600, 100, ring))
    assert bad["error"] & ref.ERR_TOKEN


def test_empty_tail_equals_no_tail():
    rng = np.random.default_rng(17)
    history, resident = 12288, 4096
    hot_valid = (rng.random(resident) > 0.1).astype(np.int32)
    lru = rng.permutation(resident)[:2048].astype(np.int64)
    reserved = ref.reserved_from_candidates(lru, resident)
    sel = np.stack([rng.permutation(history)[:TOPK] for _ in range(2)]).astype(np.int64)
    a = ref.resolve(sel, history, resident, hot_valid, reserved, lru)
    b = ref.resolve(sel, history, resident, hot_valid, reserved, lru, tail=(7000, 7000, 512))
    assert np.array_equal(a["loc"], b["loc"]) and np.array_equal(a["tokens"], b["tokens"])
    assert np.array_equal(a["changes"], b["changes"])


# ----------------------------------------------------------------------------
# Speculative windowed prefetch
# ----------------------------------------------------------------------------
def test_prefetch_windows_are_the_trigger_boundaries():
    for resident, history, windows in [(4096, 5120, 3), (16384, 131072, 8), (2048, 10240, 1), (2048, 10240, 2)]:
        ends = ref.prefetch_windows(resident, history, windows)
        assert len(ends) == windows and ends[0] == resident
        assert all(e % 128 == 0 for e in ends) and ends == sorted(ends)
        if windows >= 2:
            assert ends[-1] == history


def test_prefetch_known_answer():
    """Victim coordinates first (ordinal order, token lru[i]), then cold positions window by
    window; window and total budgets; mapped tail positions skipped; rows united."""
    resident, history = 4096, 5120            # windows 3: ends 4096, 4608, 5120
    lru = np.arange(4096 - 2048, 4096)[::-1].astype(np.int64)
    victim = np.zeros((2, 2048), bool)
    victim[0, 5] = victim[1, 7] = True
    cold = np.zeros((2, history - resident), bool)
    for t in (4100, 5000):
        cold[0, t - resident] = True
    cold[1, 4700 - resident] = True
    got = ref.prefetch(victim, cold, lru, history, resident, windows=3)
    assert got == [(int(lru[5]), 0), (int(lru[7]), 1), (4100, 2), (4700, 3), (5000, 4)]
    assert ref.prefetch(victim, cold, lru, history, resident, windows=3, window_limit=1) == \
        [(int(lru[5]), 0), (4100, 1), (4700, 2)]
    assert ref.prefetch(victim, cold, lru, history, resident, windows=3, prefetch_limit=2, window_limit=2) == \
        [(int(lru[5]), 0), (int(lru[7]), 1)]
    # 4700 is a mapped ABC tail position (first T of [4650, 4800) with T = 384)
    assert ref.prefetch(victim, cold, lru, history, resident, tail=(4650, 4800, 384), windows=3) == \
        [(int(lru[5]), 0), (int(lru[7]), 1), (4100, 2), (5000, 3)]
    assert ref.prefetch(victim, cold, lru, history, resident, windows=1, window_limit=480) == \
        [(int(lru[5]), 0), (int(lru[7]), 1)]
    with pytest.raises(ValueError):  # geometry.py:10-11: a window posts at most 480 fetches
        ref.prefetch(victim, cold, lru, history, resident, windows=1)


def _round_state(rng, history, resident, row=64):
    keys = rng.integers(0, 256, (history, 128), dtype=np.uint8)
    scales = rng.random(history).astype(np.float32)
    addresses = (np.arange(history) * row).astype(np.int64)
    logical = np.arange(history).astype(np.int64) + 1000
    pool = rng.integers(0, 256, history * row, dtype=np.uint8)
    hot = pool.reshape(history, row)[:resident].copy()
    valid = np.ones(resident, np.int32)
    return keys, scales, addresses, logical, pool, hot, valid


def test_prefetch_changes_no_output_and_keeps_residency_consistent():
    """The same TopK rows through the round with and without a prefetch: identical logical
    outputs and identical KV bytes behind every selected entry; afterwards every resident
    slot holds the KV row of the Index row at that position, and the Index rows are a
    permutation of the original ones."""
    rng = np.random.default_rng(23)
    history, resident = 8192, 4096
    for trial in range(4):
        q_rows = 1 + trial % 2
        base = _round_state(rng, history, resident)
        lru = rng.permutation(resident)[:2048].astype(np.int64)
        reserved = ref.reserved_from_candidates(lru, resident)
        sel = np.stack([rng.permutation(history)[:TOPK] for _ in range(q_rows)]).astype(np.int64)
        # Hits: most final cold selections plus unselected cold positions and victims.
        victim = rng.random((q_rows, 2048)) < 0.02
        cold = np.zeros((q_rows, history - resident), bool)
        for q in range(q_rows):
            chosen = sel[q][sel[q] >= resident] - resident
            cold[q, chosen[rng.random(len(chosen)) < 0.7]] = True
        cold |= rng.random(cold.shape) < 0.02
        pre = ref.prefetch(victim, cold, lru, history, resident, windows=4, prefetch_limit=700, window_limit=300)
        assert 0 < len(pre) <= 700
        runs = []
        for prefetched in (None, pre):
            keys, scales, addresses, logical, pool, hot, valid = (a.copy() for a in base)
            lout, sout, res, err = ref.resident_round(sel, history, resident, keys, scales, addresses, logical, valid,
                                                      reserved, lru, hot, pool, prefetched=prefetched)
            assert err == 0
            kv = np.stack([hot[sout[q]] for q in range(q_rows)])
            runs.append((lout, kv, res))
            # Residency: a valid hot slot holds the row of the Index entry now at that position.
            for p in np.nonzero(valid)[0]:
                a = int(addresses[p])
                assert np.array_equal(hot[p], pool[a:a + hot.shape[1]]), (trial, p)
            assert sorted(logical.tolist()) == sorted(base[3].tolist())
        assert np.array_equal(runs[0][0], runs[1][0])
        assert np.array_equal(runs[0][1], runs[1][1])
        # The prefetch took some of the misses off the final Fetch.
        assert len(runs[1][2]["tokens"]) < len(runs[0][2]["tokens"])
