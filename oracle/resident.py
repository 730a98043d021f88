"""CPU restatement of the resident-cache round of the streaming LIFetch resolver:
hot/cold classification of the final TopK, per-query miss resolution with LRU victim
allocation, Fetch descriptors, the Index-row permutation and the round's residency
publication. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Positions. Each request owns `history` Index rows (one per position). Position p <
`resident` is hot: its KV row lives in hot-cache slot p when hot_valid[p] != 0. TopK
selects positions; the Index update moves every fetched token's row to its new hot slot.

Follows (paths relative to the KVIP reference tree,
csrc/operators/lightning_indexer_with_fetch/op_kernel/ unless noted):
  classify   staged_topk_classify.h:9-36 (ClassifyTopkHalf), resolver_staged_dma2.h:9-22
             (StagedKnownSlot), :34-77 (StagedInitialize: Q3/Q4 same-position shortcut,
             protection bitmap of every query's hot hits); ABC tail: positions in
             [begin, end) are never hot (cache_metadata.h:22-26 IsTailToken), the first
             T = stride - resident of them are mapped to resident + kSlots + p % T at round
             start (prefetch.h:25-43 InitializeTailMappings) and ResolvePhysicalSlot
             (cache_metadata.h:102-106) turns that into ring slot resident + p % T
  resolve    resolver_staged_dma2.h:98-237 (StagedQuery): first-occurrence dedup per
             query, ranks continuing over queries, LRU candidates in ordinal order (pass 0
             ordinals >= used, pass 1 < used) skipping protected slots, fallback scan of the
             free hot slots in ascending order (lidu/op_kernel/hot_slot_selection.h:7-137
             with scan start 0), change records (record = reserved ordinal or 2048 + rank)
  events     streaming.cpp:16-22 (PublishQ: source = token position, destination = slot,
             in rank order per query), :205-274 (Consumer: batches in query order)
  init       lifecycle.cpp:32-81 (InitializeRound: changes cleared, candidate prefix of
             the change slots = the LRU candidates); reserved_hot = each candidate slot's
             LRU ordinal, as the reference harness derives it from the candidates
             (tests/operators/lifetch/support/execution.py:1557-1568)
  update     shadow_exchange_parallel.h:28-78 (ApplyBatch: 512-change chunks, closure of
             displaced rows into freed positions, freed hot positions invalidated),
             :79 (CommitMetadata: addresses / logical ids follow their rows)
  publish    common/lifetch/cache_metadata.h:54-73 (PublishDestinationResidency: every
             Fetch destination becomes valid)
  outputs    streaming.cpp:66-90 (PublishQueryOutputs) with the harness check
             tests/operators/lifetch/support/execution.py:2109-2130 (logical output =
             pre-update logical ids of the TopK positions, slot output = locations)
  failure    index_cache_update.h:5-21 (CompleteEarlyUpdate, called from
             streaming.cpp:580-583): any error of a request clears its owner's whole
             hot_valid row, so nothing partially written is trusted afterwards

Contract points that are this build's own (the reference has no counterpart): an
in-range hot slot named by two LRU candidates fails the request with ERR_CANDIDATE
before anything is resolved, and a request that fails before the Fetch publishes -1 in
both outputs (the reference publishes its outputs per query and signals errors through
status alone).

  prefetch   prefetch.h:578-832 (FastService), common/lifetch/sequence_candidates.h (the
             window's hit scan: victim coordinates [0, 2048) -> lru[i], then cold positions
             in ascending order, union over the query rows), prefetch.h:660-700
             (GatherCandidateMap + CompactMisses: already-mapped tokens skipped, the first
             `available` taken), common/lifetch/prefetch_budget.h:7-17 (PrefetchAllowance),
             python/kvip/operators/lifetch/geometry.py:4-13 (prefetch_budget), :55-61
             (trigger_tokens: window ends), prefetch.h:563-574 (PrepareCandidateWqes: slot
             resident + ordinal, mapping, RecordChange), streaming.cpp:23-27, :119-121
             (PublishPrefetch: the prefetch records are the first Index-update batch),
             streaming.cpp:330-339 (PublishPrefetchResidency)

Prefetch is restated for the case the reference reduces to when every window is serviced
after scoring has passed the window's end (its service caps each snapshot at the scheduled
boundary, prefetch.h:609-627): window 0 holds the victim candidates, window e >= 1 the cold
positions [end_{e-1}, end_e). When the service runs ahead of scoring the reference
prefetches a timing-dependent subset; the final round repairs whatever was not prefetched,
so the selected KV rows and logical outputs do not depend on it.
"""
from __future__ import annotations

import numpy as np

from oracle.lidu import ring_select

TOPK = 2048
LRU_SLOTS = 2048
CHUNK = 512
EMPTY = -1

ERR_TOKEN = 1          # a TopK position >= history
ERR_CANDIDATE = 4      # an LRU candidate >= resident, or too few free hot slots
ERR_SOURCE = 8         # a miss whose KV address is outside the host pool or not 16-byte aligned
ERR_UPDATE = 16        # an Index change that is not a valid partial permutation


def tail_slot(t, tail):
    """Ring slot of position t under tail = (begin, end, ring_slots) or None: the ABC tail
    mapping (prefetch.h:25-43) resolved by ResolvePhysicalSlot (cache_metadata.h:102-106).
    Returns (in_tail, slot or None); the slot is relative to resident."""
    if tail is None:
        return False, None
    begin, end, ring = tail
    if not begin <= t < end:
        return False, None
    return True, (t % ring if t < begin + ring else None)


def classify(selected, history, resident, hot_valid, reserved, tail=None):
    """Hot hits of every query row of one request (StagedKnownSlot, the only mapping
    entries being the ABC tail's). selected [Q, 2048] positions (-1 empty); tail =
    (begin, end, ring_slots) or None. Returns (loc [Q, 2048] with the hit slot, the ring
    slot resident + p % ring of a mapped tail position, or -1; protection bitmap as a bool
    array [resident]; error bits). Rows q >= 2 copy loc from row q - 2 where they select
    the same position at the same index. Tail bounds outside 0 <= begin <= end <= history
    set ERR_TOKEN (this build's check)."""
    q_rows = selected.shape[0]
    loc = np.full(selected.shape, EMPTY, np.int64)
    protect = np.zeros(resident, bool)
    err = 0
    if tail is not None and not 0 <= tail[0] <= tail[1] <= history:
        err |= ERR_TOKEN
        tail = None
    for q in range(q_rows):
        for i in range(TOPK):
            t = int(selected[q, i])
            if q >= 2 and t == int(selected[q - 2, i]):
                loc[q, i] = loc[q - 2, i]
                continue
            if t < 0:
                continue
            if t >= history:
                err |= ERR_TOKEN
                continue
            in_tail, ring_slot = tail_slot(t, tail)
            if in_tail:
                if ring_slot is not None:
                    loc[q, i] = resident + ring_slot
            elif t < resident and hot_valid[t] != 0 and reserved[t] < 0:
                loc[q, i] = t
                protect[t] = True
    return loc, protect, err


def prefetch_windows(resident, history, windows):
    """Window ends: trigger_tokens (geometry.py:55-61) with `windows` rounds: resident (the
    hot-ready first window), then evenly spaced 128-aligned cold boundaries up to history."""
    cold_tiles = (history - resident) // 128
    return [resident + 128 * (cold_tiles * e // max(1, windows - 1)) for e in range(windows)]


def prefetch_budget(prefetch_limit=512, window_limit=None, windows=8):
    """(prefetch_limit, window_limit) as geometry.py:4-13 derives them."""
    if window_limit is None:
        window_limit = max(1, prefetch_limit // windows)
    if not 0 <= prefetch_limit <= LRU_SLOTS or not 1 <= window_limit <= 480:
        raise ValueError("Invalid prefetch budgets: total must be 0..2048 and window 1..480")
    return prefetch_limit, window_limit


def prefetch(victim_hits, cold_hits, lru, history, resident, tail=None, windows=8, prefetch_limit=512,
             window_limit=None):
    """Speculative windowed prefetch of one request. victim_hits bool [Q, 2048]: candidate
    ordinal i scores above its row's prefix threshold; cold_hits bool [Q, >= history -
    resident]: position resident + j does (oracle.resident.prefix_classify, per query row).
    Window 0 takes victim coordinates i in order (token lru[i]); window e >= 1 the cold
    positions of [end_{e-1}, end_e) in order; a token hit by any row counts once; tokens
    already mapped (earlier windows, the ABC tail's first positions) are skipped; each
    window takes the first min(missing, PrefetchAllowance) of them. Returns [(token,
    ordinal)] in ordinal order (ordinal k is candidate slot lru[k])."""
    prefetch_limit, window_limit = prefetch_budget(prefetch_limit, window_limit, windows)
    ends = prefetch_windows(resident, history, windows)
    mapped = set()
    out = []
    victim_any = np.asarray(victim_hits, bool).any(axis=0)
    cold_any = np.asarray(cold_hits, bool).any(axis=0)
    begin = resident
    for e, end in enumerate(ends):
        if e == 0:
            cands = [int(lru[i]) for i in range(LRU_SLOTS) if victim_any[i]]
        else:
            cands = [resident + j for j in range(begin - resident, end - resident) if cold_any[j]]
            begin = end
        missing = [t for t in cands if t not in mapped and tail_slot(t, tail)[1] is None]
        used = len(out)
        # PrefetchAllowance (prefetch_budget.h:7-17): window limit, LRU slots left, prefetch
        # limit left (one request per token; no transport-queue limit here).
        available = max(0, min(window_limit, LRU_SLOTS - used, prefetch_limit - used))
        for t in missing[:available]:
            mapped.add(t)
            out.append((t, len(out)))
    return out


def resolve(selected, history, resident, hot_valid, reserved, lru, used=0, sources=None, tail=None,
            prefetched=None):
    """Per-query miss resolution of one request (StagedQuery). Returns a dict with
    loc [Q, 2048] (hot slot of every selected position, -1 for empty entries), slots
    [misses] (slot of each miss rank), tokens [misses] (position of each miss rank),
    added [Q] (new misses per query), changes / change_slots [2048 + Q*2048] records and
    the error bits. Stops (like the reference) at the first query that fails.
    sources = (addresses [history], pool_bytes, row_bytes): every new miss's KV address is
    checked against the host pool as its query is resolved (ERR_SOURCE), before any
    Fetch; this check is this build's own (the reference's transport validates its
    descriptors, cache_metadata.h:32-44). tail: the ABC tail, as for classify.
    prefetched: [(token, ordinal)] of this round's prefetch (then `used` is their count):
    a selected token that is neither a hot hit nor a mapped tail position but was
    prefetched resolves to its candidate slot lru[ordinal] and protects it
    (staged_topk_classify.h:28-31 via ResolvePhysicalSlot); its change record is the
    prefetch's (RecordChange at the ordinal) until a final miss takes that ordinal again."""
    q_rows = selected.shape[0]
    loc, protect, err = classify(selected, history, resident, hot_valid, reserved, tail)
    pmap = {} if prefetched is None else {int(t): int(k) for t, k in prefetched}
    if prefetched is not None:
        used = len(prefetched)
        for q in range(q_rows):
            for i in range(TOPK):
                t = int(selected[q, i])
                if loc[q, i] >= 0 or t not in pmap or (q >= 2 and t == int(selected[q - 2, i])):
                    continue
                s = int(lru[pmap[t]])
                if 0 <= s < resident:
                    loc[q, i] = s
                    protect[s] = True
        for q in range(2, q_rows):  # the same-position shortcut copies the resolved slot
            same = selected[q] == selected[q - 2]
            loc[q, same] = loc[q - 2, same]
    in_range = [int(s) for s in lru[:LRU_SLOTS] if 0 <= s < resident]
    if len(set(in_range)) != len(in_range):
        err |= ERR_CANDIDATE  # a hot slot named by two candidates
    bitmap = protect.copy()
    rank_of = {}
    slots, tokens, added_per_q = [], [], []
    # Round initialisation (lifecycle.cpp:58-71): no changes; the candidate prefix of
    # change_slots holds the LRU candidates.
    changes = np.full(LRU_SLOTS + q_rows * TOPK, EMPTY, np.int64)
    change_slots = np.full(LRU_SLOTS + q_rows * TOPK, EMPTY, np.int64)
    change_slots[:LRU_SLOTS] = lru[:LRU_SLOTS]
    for t, k in pmap.items():
        if not 0 <= int(lru[k]) < resident:
            err |= ERR_CANDIDATE  # a prefetch slot outside the hot range
        changes[k] = t
    for q in range(q_rows):
        if err:
            break
        # Unresolved entries, the shortcut rows excluded (they copy q - 2 at the end).
        shortcut = np.zeros(TOPK, bool)
        if q >= 2:
            shortcut = selected[q] == selected[q - 2]
        first = {}
        for i in range(TOPK):
            t = int(selected[q, i])
            if t < 0 or t >= history or shortcut[i] or loc[q, i] >= 0:
                continue
            if t in rank_of:
                continue
            first.setdefault(t, i)
        new = sorted(first.items(), key=lambda kv: kv[1])  # in index order
        old = len(slots)
        for n, (t, i) in enumerate(new):
            rank_of[t] = old + n
            tokens.append(t)
        need = len(new)
        got = []
        if need:
            # Every candidate of a pass is checked (a candidate outside the hot range
            # fails the request); the free ones are taken in ordinal order.
            for ordinals in (range(used, LRU_SLOTS), range(0, used)):
                free = []
                for o in ordinals:
                    s = int(lru[o])
                    if s >= resident or s < 0:
                        err |= ERR_CANDIDATE
                    elif not bitmap[s]:
                        free.append(s)
                got += free[:need - len(got)]
                for s in got:
                    bitmap[s] = True
                if len(got) == need:
                    break
        if len(got) < need:
            # Fallback: every known hot slot of every query is protected, then the free
            # hot slots in ascending order.
            fb = bitmap.copy()
            for s in loc.reshape(-1):
                if 0 <= s < resident:
                    fb[s] = True
            words = np.zeros((resident + 31) // 32, np.uint32)
            for s in np.nonzero(fb)[0]:
                words[s // 32] |= np.uint32(1 << (s % 32))
            extra = ring_select(words, resident, 0, need - len(got))
            if len(extra) < need - len(got):
                err |= ERR_CANDIDATE
            for s in extra:
                bitmap[s] = True
            got += list(extra)
            bitmap = bitmap | fb
        if err:
            break
        slots += got
        for i in range(TOPK):
            t = int(selected[q, i])
            if shortcut[i]:
                loc[q, i] = loc[q - 2, i]
            elif 0 <= t < history and loc[q, i] < 0:
                loc[q, i] = slots[rank_of[t]]
        for n in range(need):
            r = old + n
            s = slots[r]
            record = int(reserved[s]) if reserved[s] >= 0 else LRU_SLOTS + r
            change_slots[record] = s
            changes[record] = tokens[r]
            if sources is not None:
                addresses, pool_bytes, row_bytes = sources
                a = int(addresses[tokens[r]])
                if a < 0 or a > pool_bytes - row_bytes or a % 16:
                    err |= ERR_SOURCE
        added_per_q.append(need)
    return dict(loc=loc, slots=np.array(slots, np.int64), tokens=np.array(tokens, np.int64),
                added=np.array(added_per_q, np.int64), changes=changes, change_slots=change_slots, error=err)


def apply_changes(batches, history, resident, keys, scales, addresses, logical, hot_valid):
    """Index-row permutation of one request (ApplyBatch + CommitMetadata), in place.

    batches: list (one per query, in order) of [(orig_position, destination_slot)] in
    rank order. Row r of the tables is the row at position r before the round; a change
    moves the row of orig_position (wherever earlier changes of the round put it) to the
    destination; inside each 512-change chunk, rows displaced from destinations that are
    not themselves sources fill the freed source positions in order, and freed hot
    positions lose their residency. Returns the error bits (0 = applied)."""
    row_at = np.arange(history)
    pos_of = np.arange(history)
    addresses0, logical0 = addresses.copy(), logical.copy()
    err = _permute(batches, history, resident, keys, scales, hot_valid, row_at, pos_of)
    # Addresses and logical ids follow their rows, also for the chunks applied before a
    # rejected one.
    changed = np.nonzero(row_at != np.arange(history))[0]
    addresses[changed] = addresses0[row_at[changed]]
    logical[changed] = logical0[row_at[changed]]
    return err


def _permute(batches, history, resident, keys, scales, hot_valid, row_at, pos_of):
    """The chunk loop of apply_changes; stops at the first rejected chunk, leaving the
    earlier chunks applied. Returns the error bits."""
    for batch in batches:
        for c0 in range(0, len(batch), CHUNK):
            chunk = batch[c0:c0 + CHUNK]
            srcs, dsts = [], []
            for orig, dst in chunk:
                if not (0 <= orig < history) or not (0 <= dst < resident):
                    return ERR_UPDATE
                srcs.append(int(pos_of[orig]))
                dsts.append(int(dst))
            if len(set(srcs)) != len(srcs) or len(set(dsts)) != len(dsts):
                return ERR_UPDATE
            sset, dset = set(srcs), set(dsts)
            outs = [d for d in dsts if d not in sset]
            freed = [s for s in srcs if s not in dset]
            moves = list(zip(srcs, dsts)) + list(zip(outs, freed))
            snap_k = {s: keys[s].copy() for s, _ in moves}
            snap_s = {s: scales[s] for s, _ in moves}
            snap_row = {s: int(row_at[s]) for s, _ in moves}
            for s, d in moves:
                keys[d] = snap_k[s]
                scales[d] = snap_s[s]
                row_at[d] = snap_row[s]
                pos_of[snap_row[s]] = d
            for d in freed:
                if d < resident:
                    hot_valid[d] = 0
    return 0


def resident_round(selected, history, resident, keys, scales, addresses, logical, hot_valid, reserved, lru,
                   hot_cache, host_pool, used=0, tail=None, prefetched=None):
    """One request's full round after TopK, in place on its tables: resolve, outputs,
    Fetch (hot_cache[slot] = host_pool[addresses[token]]), Index update, residency
    publication. Returns (logical_output [Q, 2048], slot_output [Q, 2048], resolve dict,
    error bits). A failed request's owner loses all residency (hot_valid cleared); when
    it fails before the Fetch both outputs are -1 and nothing else changes. tail: the ABC
    tail (begin, end, ring_slots), as for classify. prefetched: [(token, ordinal)] of this
    round's prefetch (oracle.resident.prefetch): their rows were fetched into lru[ordinal]
    before the final resolution, they form the first Index-update batch (ordinal order,
    streaming.cpp:119-121) and every prefetch slot becomes resident (streaming.cpp:330-339)."""
    row_bytes = hot_cache.shape[1]
    pre = [] if prefetched is None else [(int(t), int(k)) for t, k in prefetched]
    for t, k in pre:  # the prefetch Fetch happens before the final resolution
        s = int(lru[k])
        a = int(addresses[t])
        if 0 <= s < resident and 0 <= a <= host_pool.size - row_bytes and a % 16 == 0:
            hot_cache[s] = host_pool[a:a + row_bytes]
    res = resolve(selected, history, resident, hot_valid, reserved, lru, used,
                  sources=(addresses, host_pool.size, hot_cache.shape[1]), tail=tail, prefetched=prefetched)
    q_rows = selected.shape[0]
    if res["error"]:
        hot_valid[:] = 0
        empty = np.full(selected.shape, EMPTY, np.int64)
        return empty, empty.copy(), res, res["error"]
    logical_out = np.full(selected.shape, EMPTY, np.int64)
    for q in range(q_rows):
        for i in range(TOPK):
            t = int(selected[q, i])
            if 0 <= t < history:
                logical_out[q, i] = logical[t]
    for t, s in zip(res["tokens"], res["slots"]):
        a = int(addresses[t])
        hot_cache[s] = host_pool[a:a + row_bytes]
    batches, r = [], 0
    if pre:
        batches.append([(t, int(lru[k])) for t, k in pre])
    for n in res["added"]:
        batches.append([(int(res["tokens"][r + k]), int(res["slots"][r + k])) for k in range(n)])
        r += n
    err = apply_changes(batches, history, resident, keys, scales, addresses, logical, hot_valid)
    if err:
        hot_valid[:] = 0
        return logical_out, res["loc"], res, err
    for s in res["slots"]:
        hot_valid[s] = 1
    for t, k in pre:
        hot_valid[int(lru[k])] = 1
    return logical_out, res["loc"], res, 0


def reserved_from_candidates(lru, resident):
    """reserved_hot of one request: the LRU ordinal of every candidate slot, -1 for the
    other hot slots (tests/operators/lifetch/support/execution.py:1557-1568)."""
    reserved = np.full(resident, EMPTY, np.int64)
    for i, s in enumerate(lru[:LRU_SLOTS]):
        if 0 <= s < resident:
            reserved[int(s)] = i
    return reserved


def prefix_classify(keys, valid, resident, lru, cold_words):
    """Resident TopK of one query row and its hit bits (ProcessResidentTopK + SaveResident,
    indexer_vector.h:100-105, :162-234; ClassifyScore / ClassifyResidentScores,
    indexer_score.h:784-792, :1018-1048; cold-tile classification, indexer_vector.h:584-593).

    keys: uint16 sortable keys of the row; valid: its valid positions. Returns
    (prefix TopK [2048] of positions [0, min(valid, resident)), threshold = the smallest
    selected key when the prefix selection is full (0 otherwise), victim bits [64] uint32
    (candidate lru[i] inside the prefix with key > threshold), cold bits [cold_words]
    uint32 (position resident + j < valid with key > threshold))."""
    from oracle.indexer import topk_reference

    pv = min(valid, resident)
    sel = topk_reference(keys, pv)
    thr = int(keys[sel].min()) if pv >= TOPK else 0
    victim = np.zeros(TOPK // 32, np.uint32)
    for i, s in enumerate(lru[:TOPK]):
        if 0 <= s < pv and int(keys[s]) > thr:
            victim[i // 32] |= np.uint32(1 << (i % 32))
    cold = np.zeros(cold_words, np.uint32)
    for j in range(max(0, valid - resident)):
        if int(keys[resident + j]) > thr:
            cold[j // 32] |= np.uint32(1 << (j % 32))
    return sel, thr, victim, cold
