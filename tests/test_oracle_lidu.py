"""Pins of the LIDU oracle (oracle/lidu.py).

* ring_select against the reference's own selector test cases and their brute-force
  expectation (tests/operators/lidu/test_hot_slot_selection.py:43-53);
* the reference KAT (tests/operators/lidu/test_lidu.py:24-79). Its fixture cannot pass
  the kernel code it exercises: its second row has no query and is not a padding row,
  which the layout check rejects (a5_lidu_fused_batch_get_prepare_mtp.cpp:1111-1133), and
  its TopK tokens map to slots inside miss_slot_bitmap, which classification treats as
  misses (:204-216). The oracle follows the kernel code; the literal fixture is checked
  to be rejected, and the KAT is run with those two points adjusted (a padding second row,
  victims outside the TopK's slots, refreshed between rounds as SlotLRU.commit does);
* a hand-computed KAT of the extended slot selection (ring scan from the cursor, hit
  slots protected, wrap, cursor update);
* the contract the reference harness verifies after every LIDU call
  (tests/operators/lifetch/support/execution.py:1478-1506) plus map invariants, checked
  on random batches from an independent classification;
* every error path: the rejected row or batch, its outputs and untouched maps.
"""
import random

import numpy as np
import pytest

from oracle import lidu as ref
from tests import lidu_cases as lc


def test_ring_select_reference_cases():
    rng = random.Random(21)
    for budget in (1, 31, 32, 33, 8192, 16384, 32768):
        for begin in (0, budget // 2, budget - 1):
            protected = {i for i in range(budget) if rng.random() < 0.65}
            free = [i for i in list(range(begin, budget)) + list(range(begin)) if i not in protected]
            n = min(len(free), 4096)
            words = [sum(1 << (i % 32) for i in protected if i // 32 == w) for w in range((budget + 31) // 32)]
            assert ref.ring_select(words, budget, begin, n) == free[:n], (budget, begin)
            assert ref.ring_select(words, budget, begin, len(free) + 5) == free  # short supply


def kat_fixture(budget, history, padding_second_row):
    batch = 2
    t2s = np.tile(np.arange(history, dtype=np.int32), (batch, 1))
    s2t = np.zeros((batch, budget), np.int32)  # execution.py:1383-1390: unmapped slots read token 0
    s2t[:, :history] = np.arange(history, dtype=np.int32)
    case = dict(
        topk=np.tile(np.arange(2048, dtype=np.int32), (4, 1)).reshape(4, 1, 2048),
        actual_seq_lengths_query=np.array([4, 4], np.int32), req_pool_entries=np.arange(batch, dtype=np.int32),
        token_to_slot=t2s, slot_to_token=s2t, eviction_cursors=np.zeros(batch, np.int32),
        cache_tokens=np.full(batch, budget, np.int32), candidate_lens=np.array([history, 0], np.int32),
        miss_slots=np.tile(np.arange(2048, dtype=np.int32), (batch, 1)),
        miss_slot_bitmap=np.zeros((batch, ref.MISS_BITMAP_WORDS), np.int32),
        resident_block_table=np.arange(batch * budget // 128, dtype=np.int32).reshape(batch, -1),
        logical_seq_lengths=np.array([history, 0], np.int32), profile_enabled=np.zeros(1, np.int32),
        layer_id=0, num_layers=1, max_num_reqs=batch, qcap=history // 128,
    )
    case["miss_slot_bitmap"][:, :64] = -1
    if padding_second_row:
        case["cache_tokens"][1] = 0
        case["logical_seq_lengths"][1] = 1
        case["req_pool_entries"][1] = batch
    return case


def test_reference_kat_fixture_is_rejected_by_the_layout_check():
    state, outs = lc.run_oracle(kat_fixture(4096, 4096, padding_second_row=False))
    assert outs["miss_counts"].tolist() == [-1, -1, 0]
    assert (outs["destination_slots"] == -1).all()


def set_victims(case, first):
    victims = np.arange(first, first + 2048, dtype=np.int32)
    case["miss_slots"][:] = victims
    case["miss_slot_bitmap"][:] = lc.bitmap_of(victims)


def test_reference_kat_adapted():
    hot = 8192
    case = kat_fixture(hot, 4096, padding_second_row=True)
    set_victims(case, 4096)  # victims are unmapped slots outside the TopK's slots
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist() == [0, 0, 0]
    assert outs["resident_seq_lengths"].tolist() == [hot, 1]
    for shift in (0, 256, 512):
        case["topk"][:] = np.arange(shift, shift + 2048, dtype=np.int32)
        state, outs = lc.run_oracle(case)
        assert outs["miss_counts"].tolist() == [0, 0, 0]
        assert np.array_equal(np.sort(outs["destination_slots"].reshape(4, 2048)), np.sort(case["topk"].reshape(4, 2048)))
    # Four disjoint source tiles with identical low token bits; four identical queries.
    history = 1 << 20
    padded = history + 20 * 128
    t2s = np.full((2, padded), -1, np.int32)
    t2s[:, :4096] = np.arange(4096, dtype=np.int32)
    case["token_to_slot"] = t2s
    case["candidate_lens"][0] = history
    case["logical_seq_lengths"][0] = history
    case["qcap"] = padded // 128
    tile = history // 4
    tokens = np.concatenate([np.arange(end - 512, end, dtype=np.int32) for end in range(tile, history + 1, tile)])
    case["topk"][:] = tokens
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist() == [2048, 0, 2048]
    slots = state["token_to_slot"][0, tokens]
    assert slots.min() >= 0 and slots.max() < hot
    assert np.array_equal(state["slot_to_token"][0, slots], tokens)
    for k in range(4):  # tile-major unique order: tile k takes victims [512k, 512k+512)
        assert set(slots[512 * k:512 * (k + 1)].tolist()) == set(range(4096 + 512 * k, 4096 + 512 * (k + 1)))
    assert np.array_equal(slots, 4096 + np.arange(2048))  # ascending inside a query (this build's order)
    assert np.array_equal(outs["indices"][:2048], tokens >> 7)
    assert np.array_equal(outs["offsets"][:2048], (tokens & 127) * 656)
    assert np.array_equal(outs["output_indices"][:2048], slots)  # identity block table
    assert (outs["indices"][2048:] == lc.SENTINEL).all()
    # The next round, with the victims refreshed, hits everything.
    case["token_to_slot"], case["slot_to_token"] = state["token_to_slot"], state["slot_to_token"]
    set_victims(case, 6144)
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist() == [0, 0, 0]


def test_extended_selection_known_answer():
    budget, cand = 4096, 32768
    t2s = np.full((1, cand), -1, np.int32)
    s2t = np.full((1, budget), -1, np.int32)
    t2s[0, 500], t2s[0, 501] = 4091, 4093
    s2t[0, 4091], s2t[0, 4093] = 500, 501
    q0 = np.concatenate(([500, 501], np.arange(10000, 12046))).astype(np.int32)
    q1 = np.concatenate((np.arange(20006, 19999, -1), np.arange(10000, 12041))).astype(np.int32)
    case = dict(
        topk=np.stack((q0, q1)).reshape(2, 1, 2048), actual_seq_lengths_query=np.array([2], np.int32),
        req_pool_entries=np.zeros(1, np.int32), token_to_slot=t2s, slot_to_token=s2t,
        eviction_cursors=np.array([4090], np.int32), cache_tokens=np.array([budget], np.int32),
        candidate_lens=np.array([cand], np.int32), miss_slots=np.arange(2048, dtype=np.int32)[None],
        miss_slot_bitmap=lc.bitmap_of(range(2048))[None], resident_block_table=np.arange(32, dtype=np.int32)[None],
        logical_seq_lengths=np.array([cand + 3], np.int32), profile_enabled=np.zeros(1, np.int32),
        layer_id=0, num_layers=1, max_num_reqs=1, qcap=cand // 128,
    )
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist() == [2053, 2053]
    fwd = state["token_to_slot"][0]
    assert np.array_equal(fwd[10000:12046], np.arange(2046))
    assert fwd[20000] == 2046 and fwd[20001] == 2047
    assert fwd[20002:20007].tolist() == [4090, 4092, 4094, 4095, 2048]
    assert state["eviction_cursors"].tolist() == [2049]
    assert fwd[500] == 4091 and fwd[501] == 4093
    dest = outs["destination_slots"].reshape(2, 2048)
    assert dest[0, -2:].tolist() == [4091, 4093] and dest[0, 0] == 0
    assert dest[1, :7].tolist() == [2048, 4095, 4094, 4092, 4090, 2047, 2046]
    assert outs["resident_seq_lengths"].tolist() == [budget + 3]


def independent_contract(case, state, outs):
    """The reference harness's post-conditions (execution.py:1478-1506) and map
    invariants, from a classification computed here, not by the oracle."""
    batch = len(case["actual_seq_lengths_query"])
    dummy = int(case["profile_enabled"][0]) == ref.PROFILE_MODE_GRAPH_DUMMY
    counts = outs["miss_counts"]
    dest = outs["destination_slots"].reshape(-1, 2048)
    prefix = 0
    touched = set()
    for r in range(batch):
        q0 = 0 if r == 0 else int(case["actual_seq_lengths_query"][r - 1])
        qn = int(case["actual_seq_lengths_query"][r]) - q0
        pool, budget, cand = (int(case[k][r]) for k in ("req_pool_entries", "cache_tokens", "candidate_lens"))
        if counts[r] < 0 or budget == 0:
            assert (dest[q0:q0 + qn] == -1).all()
            if counts[r] < 0:
                assert outs["resident_seq_lengths"][r] == 0
            continue
        touched.add(pool)
        before = case["token_to_slot"][pool]
        after = state["token_to_slot"][pool]
        words = np.zeros(ref.MISS_BITMAP_WORDS, np.uint32) if dummy else case["miss_slot_bitmap"][r].view(np.uint32)
        misses, hits = set(), set()
        for q in range(qn):
            toks = case["topk"][q0 + q, 0].astype(np.int64)
            if dummy:
                toks = np.where((toks < 0) | (toks >= cand), 0, toks)
            for t in toks:
                m = int(before[t])
                (hits if 0 <= m < budget and not (int(words[m >> 5]) >> (m & 31)) & 1 else misses).add(int(t))
            got = np.sort(dest[q0 + q])
            assert np.array_equal(got, np.sort(after[toks])), (r, q)
            assert got.min() >= 0 and got.max() < budget
            assert np.array_equal(state["slot_to_token"][pool, after[toks]], toks)
        assert int(counts[r]) == len(misses)
        for t in hits:
            assert after[t] == before[t]
        new_slots = {int(after[t]) for t in misses}
        assert len(new_slots) == len(misses)
        victims = case["miss_slots"][r, :min(len(misses), 2048)]
        assert set(victims.tolist()) <= new_slots
        assert not new_slots & {int(before[t]) for t in hits}
        mapped = after[after >= 0]
        assert len(np.unique(mapped)) == len(mapped)  # forward map stays injective
        d_idx = outs["indices"][prefix:prefix + len(misses)]
        d_off = outs["offsets"][prefix:prefix + len(misses)]
        d_out = outs["output_indices"][prefix:prefix + len(misses)]
        base = (pool * case["num_layers"] + case["layer_id"]) * case["qcap"]
        toks = (d_idx.astype(np.int64) - base) * 128 + d_off // 656
        assert set(toks.tolist()) == misses
        table = case["resident_block_table"][r]
        slots = after[toks]
        assert np.array_equal(d_out, table[slots >> 7] * 128 + (slots & 127))
        prefix += len(misses)
        logical = int(case["logical_seq_lengths"][r])
        assert outs["resident_seq_lengths"][r] == (budget + logical - cand if logical >= cand else 0)
    assert counts[batch] == prefix
    for pool in range(case["token_to_slot"].shape[0]):
        if pool not in touched:
            assert np.array_equal(state["token_to_slot"][pool], case["token_to_slot"][pool])
            assert np.array_equal(state["slot_to_token"][pool], case["slot_to_token"][pool])


@pytest.mark.parametrize("seed,queries,kw", [
    (1, (1, 2, 4), {}),
    (2, (4, 4), dict(hot_tokens=8192, hit_share=0.3, budget=8192)),
    (3, (3, 1, 2, 4), dict(cand=(1 << 20) + 1000, hot_tokens=4096)),
    (4, (2, 2), dict(trailing=3)),
    (5, (4,), dict(hot_tokens=2048, hit_share=1.0)),
    (6, (4, 2), dict(hot_tokens=8192, hit_share=0.0, budget=12288, cand=40000)),
])
def test_contract_on_random_batches(seed, queries, kw):
    case = lc.random_case(seed, queries=queries, **kw)
    state, outs = lc.run_oracle(case)
    assert (outs["miss_counts"][:-1] >= 0).all()
    independent_contract(case, state, outs)
    packed = int(case["actual_seq_lengths_query"][-1])
    assert (outs["destination_slots"][packed:] == lc.SENTINEL).all()


def test_padding_rows_and_graph_dummy_mode():
    case = lc.add_padding_row(lc.add_padding_row(lc.random_case(7, queries=(2, 1)), queries=2), queries=0)
    case["topk"][0, 0, :5] = [-1, -1, 5, case["candidate_lens"][0] + 3, -1]
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist()[:2] == [-1, outs["miss_counts"][1]] and outs["miss_counts"][1] >= 0
    assert outs["miss_counts"][2] == 0 and outs["miss_counts"][3] == 0
    assert outs["resident_seq_lengths"][2] == 1
    independent_contract(case, state, outs)
    # Graph-dummy mode (the warm-up of a captured graph) ignores the victim bitmap, so a
    # hit may sit on a slot that the same round hands to a miss: only the classification
    # and the counts are checked there.
    case["profile_enabled"][0] = ref.PROFILE_MODE_GRAPH_DUMMY
    state, outs = lc.run_oracle(case)
    assert (outs["miss_counts"][:-1] >= 0).all()
    dest = outs["destination_slots"].reshape(-1, 2048)
    for r in range(2):
        q0 = 0 if r == 0 else int(case["actual_seq_lengths_query"][r - 1])
        pool, budget, cand = (int(case[k][r]) for k in ("req_pool_entries", "cache_tokens", "candidate_lens"))
        misses = set()
        for q in range(q0, int(case["actual_seq_lengths_query"][r])):
            toks = case["topk"][q, 0].astype(np.int64)
            toks = np.where((toks < 0) | (toks >= cand), 0, toks)
            before = case["token_to_slot"][pool, toks]
            hit = (before >= 0) & (before < budget)
            misses |= set(toks[~hit].tolist())
            assert np.array_equal(dest[q, hit.size - hit.sum():], before[hit])  # hit suffix in TopK order
        assert outs["miss_counts"][r] == len(misses)


def rejected_row(case, r, state, outs):
    pool = int(case["req_pool_entries"][r])
    assert outs["miss_counts"][r] == -1 and outs["resident_seq_lengths"][r] == 0
    q0 = 0 if r == 0 else int(case["actual_seq_lengths_query"][r - 1])
    q1 = int(case["actual_seq_lengths_query"][r])
    assert (outs["destination_slots"][q0:q1] == -1).all()
    assert np.array_equal(state["token_to_slot"][pool], case["token_to_slot"][pool])
    assert np.array_equal(state["slot_to_token"][pool], case["slot_to_token"][pool])
    assert state["eviction_cursors"][pool] == case["eviction_cursors"][pool]


def test_row_errors_leave_other_rows_working():
    base = lc.random_case(8, queries=(2, 2, 2), hot_tokens=8192, hit_share=0.2, budget=6144)
    edits = {
        "metadata": lambda c: c["cache_tokens"].__setitem__(1, 2047),
        "topk_token": lambda c: c["topk"].__setitem__((2, 0, 7), -1),
        "destination": lambda c: c["miss_slots"].__setitem__((1, 3), c["cache_tokens"][1]),
        "resident_block": lambda c: c["resident_block_table"].__setitem__((1, slice(None)), -1),
        "insufficient": lambda c: (c["cache_tokens"].__setitem__(1, 2200),
                                   c["miss_slots"].__setitem__(1, np.arange(2048)),
                                   c["miss_slot_bitmap"].__setitem__(1, lc.bitmap_of(range(2048)))),
    }
    for name, edit in edits.items():
        case = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in base.items()}
        edit(case)
        state, outs = lc.run_oracle(case)
        rejected_row(case, 1, state, outs)
        assert outs["miss_counts"][0] >= 0 and outs["miss_counts"][2] >= 0, name
        independent_contract(case, state, outs)


@pytest.mark.parametrize("edit", ["alias", "too_many", "beyond_packed", "empty_row"])
def test_batch_rejections(edit):
    case = lc.random_case(9, queries=(2, 2, 1), trailing=2)
    if edit == "alias":
        case["req_pool_entries"][2] = case["req_pool_entries"][0]
    elif edit == "too_many":
        case["actual_seq_lengths_query"][:] = [5, 6, 7]
    elif edit == "beyond_packed":
        case["actual_seq_lengths_query"][2] = case["topk"].shape[0] + 1
    else:
        case["actual_seq_lengths_query"][1] = case["actual_seq_lengths_query"][0]
    state, outs = lc.run_oracle(case)
    assert outs["miss_counts"].tolist() == [-1, -1, -1, 0]
    assert (outs["destination_slots"] == -1).all()  # every packed row, the trailing ones too
    assert (outs["resident_seq_lengths"] == 0).all()
    for k in lc.STATE:
        assert np.array_equal(state[k], case[k])
