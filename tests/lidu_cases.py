"""LIDU inputs shared by the oracle tests and the GPU parity tests: consistent resident
maps per pool row, victim slots with their bitmap, TopK rows with a chosen hit/miss mix
and overlap between the queries of one request."""
from __future__ import annotations

import numpy as np

from oracle import lidu as ref

SENTINEL = -7  # output entries the operator must leave untouched keep this value


def empty_outputs(packed, batch):
    cap = batch * ref.MISS_CAP
    return dict(
        destination_slots=np.full((packed, 1, ref.SPARSE), SENTINEL, np.int32),
        miss_counts=np.full(batch + 1, SENTINEL, np.int32),
        indices=np.full(cap, SENTINEL, np.int32),
        offsets=np.full(cap, SENTINEL, np.int32),
        output_indices=np.full(cap, SENTINEL, np.int32),
        resident_seq_lengths=np.full(batch, SENTINEL, np.int32),
    )


def bitmap_of(slots, words=ref.MISS_BITMAP_WORDS):
    bits = np.zeros(words, np.uint32)
    for s in slots:
        if 0 <= s < 32 * words:
            bits[s >> 5] |= np.uint32(1) << np.uint32(s & 31)
    return bits.view(np.int32)


def random_case(seed, *, queries=(1, 2, 4), budget=4096, cand=16384, resident_fill=0.9, hot_tokens=3072,
                hit_share=0.7, stale=16, extra_pool_rows=2, trailing=0, layer_id=1, num_layers=3):
    """One request per entry of `queries` (its query count). Per request: `budget` resident
    slots, `resident_fill` of them mapped to random tokens of [0, cand); 2048 random victim
    slots; every query draws 2048 distinct tokens from a request hot set of `hot_tokens`
    tokens of which `hit_share` are resident."""
    rng = np.random.default_rng(seed)
    batch = len(queries)
    budgets = np.broadcast_to(np.asarray(budget), (batch,)).astype(np.int64)
    cands = np.broadcast_to(np.asarray(cand), (batch,)).astype(np.int64)
    pool_size = batch + extra_pool_rows
    source_cap = int((cands.max() + 127) // 128 * 128)
    resident_cap = int(budgets.max())
    res_blocks = int((resident_cap + 127) // 128) + 1
    t2s = np.full((pool_size, source_cap), -1, np.int32)
    s2t = np.full((pool_size, resident_cap), -1, np.int32)
    cursors = rng.integers(-1, resident_cap, pool_size).astype(np.int32)
    pool_rows = rng.permutation(pool_size)[:batch].astype(np.int32)
    ends = np.cumsum(queries).astype(np.int32)
    packed = int(ends[-1]) + trailing
    topk = np.full((packed, 1, ref.SPARSE), -1, np.int32)
    miss_slots = np.zeros((batch, ref.SPARSE), np.int32)
    bitmap = np.zeros((batch, ref.MISS_BITMAP_WORDS), np.int32)
    block_table = np.zeros((batch, res_blocks), np.int32)
    for row in range(pool_size):  # rows outside the batch hold state that must survive
        n = int(min(budgets.min(), cands.min()) * resident_fill)
        toks = rng.choice(source_cap, n, replace=False)
        slots = rng.choice(resident_cap, n, replace=False)
        t2s[row, toks] = slots
        s2t[row, slots] = toks
    for b in range(batch):
        pool, bud, cnd = int(pool_rows[b]), int(budgets[b]), int(cands[b])
        t2s[pool] = -1
        s2t[pool] = -1
        n_res = int(min(bud, cnd) * resident_fill)
        res_tokens = rng.choice(cnd, n_res, replace=False)
        res_slots = rng.choice(bud, n_res, replace=False)
        t2s[pool, res_tokens] = res_slots
        s2t[pool, res_slots] = res_tokens
        # Stale reverse entries: the slot names a token whose forward entry points elsewhere.
        free = np.setdiff1d(np.arange(bud), res_slots)
        for s in rng.choice(free, min(stale, len(free)), replace=False):
            s2t[pool, s] = int(rng.choice(res_tokens))
        victims = rng.choice(bud, ref.SPARSE, replace=False).astype(np.int32)
        miss_slots[b] = victims
        bitmap[b] = bitmap_of(victims)
        block_table[b] = rng.choice(1 << 20, res_blocks, replace=False)
        n_hot_res = min(int(hot_tokens * hit_share), n_res)
        non_res = np.setdiff1d(rng.choice(cnd, min(cnd, 4 * hot_tokens), replace=False), res_tokens)
        hot = np.concatenate((rng.choice(res_tokens, n_hot_res, replace=False),
                              non_res[:hot_tokens - n_hot_res]))
        q0 = 0 if b == 0 else int(ends[b - 1])
        for q in range(queries[b]):
            topk[q0 + q, 0] = rng.permutation(rng.choice(hot, ref.SPARSE, replace=False))
    logical = (cands + rng.integers(0, 200, batch)).astype(np.int32)
    return dict(
        topk=topk, actual_seq_lengths_query=ends, req_pool_entries=pool_rows, token_to_slot=t2s,
        slot_to_token=s2t, eviction_cursors=cursors, cache_tokens=budgets.astype(np.int32),
        candidate_lens=cands.astype(np.int32), miss_slots=miss_slots, miss_slot_bitmap=bitmap,
        resident_block_table=block_table, logical_seq_lengths=logical,
        profile_enabled=np.zeros(1, np.int32), layer_id=layer_id, num_layers=num_layers,
        max_num_reqs=pool_size, qcap=(source_cap + 127) // 128,
    )


def add_padding_row(case, queries=0):
    """Append a graph padding row (:1303-1320) with `queries` query rows."""
    c = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in case.items()}
    end = int(c["actual_seq_lengths_query"][-1]) + queries
    c["actual_seq_lengths_query"] = np.append(c["actual_seq_lengths_query"], end).astype(np.int32)
    packed = max(c["topk"].shape[0], end)
    if packed > c["topk"].shape[0]:
        pad = np.zeros((packed - c["topk"].shape[0], 1, ref.SPARSE), np.int32)
        c["topk"] = np.concatenate((c["topk"], pad))
    c["req_pool_entries"] = np.append(c["req_pool_entries"], c["max_num_reqs"]).astype(np.int32)
    for name, value in (("cache_tokens", 0), ("candidate_lens", 0), ("logical_seq_lengths", 1)):
        c[name] = np.append(c[name], value).astype(np.int32)
    c["miss_slots"] = np.concatenate((c["miss_slots"], np.zeros((1, ref.SPARSE), np.int32)))
    c["miss_slot_bitmap"] = np.concatenate((c["miss_slot_bitmap"], np.zeros((1, ref.MISS_BITMAP_WORDS), np.int32)))
    c["resident_block_table"] = np.concatenate(
        (c["resident_block_table"], np.zeros((1, c["resident_block_table"].shape[1]), np.int32)))
    return c


INPUTS = ("topk", "actual_seq_lengths_query", "req_pool_entries", "token_to_slot", "slot_to_token",
          "eviction_cursors", "cache_tokens", "candidate_lens", "miss_slots", "miss_slot_bitmap",
          "resident_block_table", "logical_seq_lengths", "profile_enabled")
OUTPUTS = ("destination_slots", "miss_counts", "indices", "offsets", "output_indices", "resident_seq_lengths")
STATE = ("token_to_slot", "slot_to_token", "eviction_cursors")


def run_oracle(case):
    """Copy of the case run through oracle/lidu.py; returns (state, outputs) dicts."""
    state = {k: case[k].copy() for k in STATE}
    outs = empty_outputs(case["topk"].shape[0], len(case["actual_seq_lengths_query"]))
    args = [state[k] if k in state else case[k] for k in INPUTS]
    ref.lidu(*args, *[outs[k] for k in OUTPUTS], case["layer_id"], case["num_layers"], case["max_num_reqs"],
             case["qcap"])
    return state, outs
