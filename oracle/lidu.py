"""CPU restatement of the LIDU operator (kvip.lidu): TopK classification against the
resident maps, miss-first compaction, request-level miss deduplication, slot selection,
victim clearing, map installation, miss-prefix refill and BatchGet descriptors.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows csrc/operators/lidu/op_kernel/a5_lidu_fused_batch_get_prepare_mtp.cpp:
batch flow :674-813, layout check :1111-1149, row validity :1290-1329, classification
:195-221 + compaction :1381-1449, dedup :223-262 + :1986-2021 + :1497-1521, extended slot
selection :1564-1741 with op_kernel/hot_slot_selection.h, destination validation :264-295 +
:1743-1797, clear :350-386, install :388-424, refill :426-449, descriptors :451-545 +
:2198-2261, batch outputs :2111-2196. Host shape checks: torch_extension/csrc/
lidu_fused_batch_get_prepare_mtp_ops.cpp:41-190.

Deduplication order. The reference walks source tiles of 2^18 tokens, and inside a tile
the queries in order; within one query it assigns unique-miss ordinals with SIMT atomics
(:223-262), so that order is not fixed by the reference. This restatement and the device
kernel emit each query's new tokens of a tile in ascending token order, which is one of
the orders the reference can produce; the unique set, its tile/query grouping, every map
outcome and every count are independent of that choice.
"""
from __future__ import annotations

import numpy as np

SPARSE = 2048
MAX_Q = 4
MISS_CAP = SPARSE * MAX_Q
MAX_SOURCE = (1 << 20) + 20 * 128
MAX_CACHE = (1 << 17) + 20 * 128
MISS_BITMAP_WORDS = ((MAX_CACHE + 31) // 32 + 7) // 8 * 8
SOURCE_TILE = 1 << 18
ROW_BYTES = 656

OK = 0
ERROR_QUERY_LAYOUT = -100
ERROR_ROW_METADATA = -101
ERROR_DUPLICATE_POOL_ROW = -102
ERROR_TOPK_TOKEN = -103
ERROR_UNIQUE_MISS_CAPACITY = -106
ERROR_INSUFFICIENT_EVICTION_SLOTS = -107
ERROR_RESOLVED_SLOT = -109
ERROR_DESTINATION_SLOT = -110
ERROR_RESIDENT_BLOCK = -111
PROFILE_MODE_GRAPH_DUMMY = 2


def ring_select(protected_words, budget, scan_begin, count):
    """Up to `count` slots whose protected bit is clear, scanning bitmap words in ring
    order: words of [scan_begin, budget), then words of [0, scan_begin), each masked to
    its segment, bits ascending (:1632-1725, op_kernel/hot_slot_selection.h:7-137)."""
    first = (budget - 1) // 32 - scan_begin // 32 + 1
    second = (scan_begin - 1) // 32 + 1 if scan_begin else 0
    out = []
    for o in range(first + second):
        if o < first:
            w, lo, hi = scan_begin // 32 + o, scan_begin, budget
        else:
            w, lo, hi = o - first, 0, scan_begin
        base = 32 * w
        mask = 0xFFFFFFFF
        if lo > base:
            mask &= (0xFFFFFFFF << (lo - base)) & 0xFFFFFFFF
        if hi < base + 32:
            mask &= (1 << (hi - base)) - 1
        available = ~int(protected_words[w]) & mask
        while available and len(out) < count:
            low = available & -available
            out.append(base + low.bit_length() - 1)
            available ^= low
    return out


def _bit(words, slot):
    return (int(words[slot >> 5]) >> (slot & 31)) & 1


def _words(array_row):
    return np.asarray(array_row, np.int64).astype(np.uint32)


def lidu(topk, actual_seq_lengths_query, req_pool_entries, token_to_slot, slot_to_token, eviction_cursors,
         cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table, logical_seq_lengths,
         profile_enabled, destination_slots, miss_counts, indices, offsets, output_indices, resident_seq_lengths,
         layer_id, num_layers, max_num_reqs, qcap):
    """The out-variant on numpy int32 arrays, argument order of the reference ABI
    (python/kvip/operators/lidu.py:4-8). token_to_slot, slot_to_token, eviction_cursors and
    the six outputs are updated in place; output entries the reference does not write
    (query rows past the last request, descriptors past the total) keep their values."""
    packed = topk.shape[0]
    tk = np.asarray(topk).reshape(packed, SPARSE)
    dest = destination_slots.reshape(packed, SPARSE)
    batch = len(actual_seq_lengths_query)
    pool_size, source_cap = token_to_slot.shape
    resident_cap = slot_to_token.shape[1]
    res_blocks = resident_block_table.shape[1]
    graph_dummy = int(profile_enabled[0]) == PROFILE_MODE_GRAPH_DUMMY

    def padding_row(r):
        return (int(cache_tokens[r]) == 0 and int(candidate_lens[r]) == 0 and int(logical_seq_lengths[r]) == 1
                and int(req_pool_entries[r]) == max_num_reqs)

    # Query layout and pool-row aliasing (:1111-1149): any failure rejects the batch.
    layout_ok = True
    previous = 0
    for r in range(batch):
        end = int(actual_seq_lengths_query[r])
        count = end - previous
        if previous < 0 or end < previous or end > packed or (count < 1 and not padding_row(r)) or count > MAX_Q:
            layout_ok = False
        previous = end
    for r in range(batch):
        for p in range(r):
            if int(req_pool_entries[r]) == int(req_pool_entries[p]) and not (padding_row(r) and padding_row(p)):
                layout_ok = False
    if not layout_ok:
        dest[:] = -1
        miss_counts[:batch] = -1
        miss_counts[batch] = 0
        resident_seq_lengths[:] = 0
        return

    rows = []
    for r in range(batch):
        q0 = 0 if r == 0 else int(actual_seq_lengths_query[r - 1])
        qn = int(actual_seq_lengths_query[r]) - q0
        budget, cand, pool = int(cache_tokens[r]), int(candidate_lens[r]), int(req_pool_entries[r])
        valid = (SPARSE <= budget <= MAX_CACHE and budget <= resident_cap and SPARSE <= cand <= source_cap
                 and (cand + 127) // 128 <= qcap and (budget + 127) // 128 <= res_blocks
                 and 0 <= pool < pool_size and pool < max_num_reqs)
        pad = padding_row(r)
        row = dict(status=OK if (valid or pad) else ERROR_ROW_METADATA, q0=q0, qn=qn, budget=budget, cand=cand,
                   pool=pool, unique=[], slots=[], resolved=False, cursor=-1, misses=[[] for _ in range(qn)])
        rows.append(row)
        if pad or row["status"] != OK:
            dest[q0:q0 + qn] = -1
            continue
        membership = np.zeros(MISS_BITMAP_WORDS, np.uint32) if graph_dummy else _words(miss_slot_bitmap[r])
        protected = membership.copy()
        for q in range(qn):
            toks = tk[q0 + q].astype(np.int64).copy()
            if graph_dummy:
                toks[(toks < 0) | (toks >= cand)] = 0
            cls = np.full(SPARSE, -1, np.int64)
            for i, t in enumerate(toks):
                if 0 <= t < cand:
                    m = int(token_to_slot[pool, t])
                    if 0 <= m < budget and not _bit(membership, m):
                        cls[i] = m
            miss = toks[cls < 0]
            hits = cls[cls >= 0]
            dest[q0 + q] = np.concatenate((np.full(len(miss), -1, np.int64), hits)).astype(np.int32)
            row["misses"][q] = [int(t) for t in miss]
            for s in hits:
                protected[s >> 5] |= np.uint32(1) << np.uint32(s & 31)
        status = OK
        if any(t < 0 or t >= cand for q in range(qn) for t in row["misses"][q]):
            status = ERROR_TOPK_TOKEN
        unique = row["unique"]
        if status == OK and any(row["misses"]):
            seen = set()
            for tile in range(0, cand, SOURCE_TILE):
                for q in range(qn):
                    fresh = sorted({t for t in row["misses"][q] if tile <= t < tile + SOURCE_TILE} - seen)
                    seen.update(fresh)
                    unique.extend(fresh)
        if status == OK and len(unique) > MISS_CAP:
            status = ERROR_UNIQUE_MISS_CAPACITY
        slots = [int(s) for s in miss_slots[r][:min(len(unique), SPARSE)]]
        if status == OK and len(unique) > SPARSE:
            cur = int(eviction_cursors[pool])
            begin = cur % budget if cur >= 0 else 0
            extra = ring_select(protected, budget, begin, len(unique) - SPARSE)
            if len(extra) != len(unique) - SPARSE:
                status = ERROR_INSUFFICIENT_EVICTION_SLOTS
            else:
                slots += extra
                row["resolved"] = True
                row["cursor"] = 0 if extra[-1] + 1 == budget else extra[-1] + 1
        if status == OK and unique:
            if any(s < 0 or s >= budget or (s >> 7) >= res_blocks for s in slots):
                status = ERROR_DESTINATION_SLOT
            elif any(not 0 <= int(resident_block_table[r][s >> 7]) <= 0x7FFFFFFF // 128 for s in slots):
                status = ERROR_RESIDENT_BLOCK
        row["slots"] = slots
        if status != OK:
            dest[q0:q0 + qn] = -1
        row["status"] = status

    def live(row):
        return row["status"] == OK and 0 < len(row["unique"]) <= MISS_CAP

    # Every request's victims are cleared before any install (:773-790).
    for row in filter(live, rows):
        pool, cand = row["pool"], row["cand"]
        for s in row["slots"]:
            if 0 <= s < resident_cap:
                victim = int(slot_to_token[pool, s])
                if 0 <= victim < cand and int(token_to_slot[pool, victim]) == s:
                    token_to_slot[pool, victim] = -1
    for row in filter(live, rows):
        pool, cand, budget = row["pool"], row["cand"], row["budget"]
        for t, s in zip(row["unique"], row["slots"]):
            if 0 <= s < resident_cap:
                if 0 <= t < cand:
                    token_to_slot[pool, t] = s
                if s < budget:
                    slot_to_token[pool, s] = t
    total = 0
    for r, row in enumerate(rows):
        if live(row):
            for q in range(row["qn"]):
                for i, t in enumerate(row["misses"][q]):
                    dest[row["q0"] + q, i] = token_to_slot[row["pool"], t]
            base = (row["pool"] * num_layers + layer_id) * qcap
            for c, (t, s) in enumerate(zip(row["unique"], row["slots"])):
                o = total + c
                indices[o] = np.int64(base + (t >> 7)).astype(np.uint32).astype(np.int32)
                offsets[o] = (t & 127) * ROW_BYTES
                out = -1
                if s < resident_cap and (s >> 7) < res_blocks:
                    pb = int(resident_block_table[r][s >> 7])
                    if 0 <= pb <= 0x7FFFFFFF // 128:
                        out = pb * 128 + (s & 127)
                output_indices[o] = out
            total += len(row["unique"])
        ok = row["status"] == OK
        miss_counts[r] = len(row["unique"]) if ok else -1
        if ok and row["resolved"] and row["pool"] >= 0 and row["cursor"] >= 0:
            eviction_cursors[row["pool"]] = row["cursor"]
        resident_seq_lengths[r] = 0
        if ok:
            budget, cand, logical = row["budget"], row["cand"], int(logical_seq_lengths[r])
            if budget >= SPARSE and cand >= SPARSE and logical >= cand:
                resident_seq_lengths[r] = (budget + logical - cand + (1 << 31)) % (1 << 32) - (1 << 31)
            elif budget == 0 and logical >= 0:
                resident_seq_lengths[r] = logical
    miss_counts[batch] = total
