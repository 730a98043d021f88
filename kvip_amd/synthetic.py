"""Seeded synthetic decode workloads at the benchmark shapes (no datasets, no network).

`decode_workload` builds, directly on the device, everything one LIFetch decode round
reads: request context lengths, a shuffled block table, a paged index-K cache with
per-token scales, the index queries and head weights, and a paged KV cache of
656-byte rows filled with random bytes (any misplaced byte is detectable).

Configurations (the benchmark configurations):
  c1: batch 4, ctx 4096, bf16 Q/K ~N(0,1), fp32 weights ~N(0,1)/8, no scales.
  c2: batch 64, ctx ~U{8192..32768}, fp8 e4m3 Q/K from N(0,1) (saturating cast),
      per-token key scale ~U(0.5, 2), fp32 weights ~N(0,1)/8, KV rows of 656 bytes.
  c3 (`prefill_workload`): one sequence, 4096 query rows against 65536 context tokens,
      right-down causal (row i sees 61440 + i + 1 tokens), fp8 Q/K from N(0,1), per-row
      query scales ~U(0.5, 1.5) and per-token key scales ~U(0.5, 2), fp32 weights
      ~N(0,1)/8; the new rows' index-K sit at the sequence's last 4096 paged slots.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

BLOCK_TOKENS = 128
INDEX_DIM = 128


@dataclass
class DecodeWorkload:
    ctx: np.ndarray            # [batch] context tokens per request
    block_table: object        # torch int32 [batch, max_blocks]
    keys: object               # torch [num_blocks, 128, 128] fp8 e4m3 / bf16
    key_scale: object          # torch float32 [num_blocks, 128] or None
    query: object              # torch [rows, heads, 128]
    weights: object            # torch [rows, heads]
    query_scale: object        # torch float32 [rows, heads] or None
    kv_cache: object           # torch uint8 [num_blocks, 128, row_bytes] or None
    rows_per_request: int
    seed: int

    @property
    def batch(self):
        return len(self.ctx)

    @property
    def max_blocks(self):
        return int(self.block_table.shape[1])


def saturating_fp8(torch, x):
    return x.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def decode_workload(torch, *, batch, device, ctx=None, ctx_low=None, ctx_high=None, heads=64, qk="fp8",
                    weight_dtype=None, key_scale=True, query_scale=False, rows_per_request=1,
                    kv_row_bytes=656, seed=0, max_context=None):
    rng = np.random.default_rng(seed)
    if ctx is None:
        ctx = rng.integers(ctx_low, ctx_high + 1, size=batch)
    ctx = np.asarray(ctx, dtype=np.int64)
    blocks_per = (ctx + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    max_ctx = int(max_context or max(int(ctx.max()), 1))
    max_blocks = (max_ctx + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    num_blocks = max(int(blocks_per.sum()), 1)
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.zeros((batch, max_blocks), np.int32)
    offset = 0
    for b, n in enumerate(blocks_per):
        table[b, :n] = perm[offset:offset + n]
        offset += n
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dev = torch.device(device)
    rows = batch * rows_per_request
    weight_dtype = torch.float32 if weight_dtype is None else weight_dtype

    def normal(shape):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)

    if qk == "fp8":
        keys = saturating_fp8(torch, normal((num_blocks, BLOCK_TOKENS, INDEX_DIM)))
        query = saturating_fp8(torch, normal((rows, heads, INDEX_DIM)))
    else:
        keys = normal((num_blocks, BLOCK_TOKENS, INDEX_DIM)).to(torch.bfloat16)
        query = normal((rows, heads, INDEX_DIM)).to(torch.bfloat16)
    weights = (normal((rows, heads)) / 8).to(weight_dtype)
    ks = None
    if key_scale:
        ks = torch.rand((num_blocks, BLOCK_TOKENS), generator=gen, device=dev, dtype=torch.float32) * 1.5 + 0.5
    qs = None
    if query_scale:
        qs = torch.rand((rows, heads), generator=gen, device=dev, dtype=torch.float32) + 0.5
    kv = None
    if kv_row_bytes:
        kv = torch.randint(0, 256, (num_blocks, BLOCK_TOKENS, kv_row_bytes), generator=gen, device=dev,
                           dtype=torch.uint8)
    return DecodeWorkload(ctx=ctx, block_table=torch.from_numpy(table).to(dev), keys=keys, key_scale=ks,
                          query=query, weights=weights, query_scale=qs, kv_cache=kv,
                          rows_per_request=rows_per_request, seed=seed)


def config_workload(torch, name, device, seed=2026):
    """The benchmark configurations by name ('c1' or 'c2')."""
    if name == "c1":
        return decode_workload(torch, batch=4, ctx=[4096] * 4, device=device, qk="bf16", key_scale=False,
                               seed=seed)
    if name == "c2":
        return decode_workload(torch, batch=64, ctx_low=8192, ctx_high=32768, device=device, qk="fp8",
                               key_scale=True, seed=seed, max_context=32768)
    raise ValueError(f"unknown decode configuration {name!r}")


def prefill_workload(torch, device, *, seed=2026, q_len=4096, k_len=65536, heads=64, qk="fp8"):
    """Config-3 prefill chunk on the device: dict of the PrefillIndexer inputs plus the
    slot_mapping [q_len] int64 and target positions [q_len] int64 of the new rows. qk:
    "fp8" (e4m3 Q/K with per-row query and per-token key scales) or "bf16" (no scales)."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dev = torch.device(device)
    blocks = (k_len + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    table = rng.permutation(blocks).astype(np.int32)[None, :]

    def normal(shape):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)

    if qk not in ("fp8", "bf16"):
        raise ValueError(f"qk must be fp8 or bf16 (got {qk})")
    cast = (lambda x: saturating_fp8(torch, x)) if qk == "fp8" else (lambda x: x.to(torch.bfloat16))
    keys = cast(normal((blocks, BLOCK_TOKENS, INDEX_DIM)))
    query = cast(normal((q_len, heads, INDEX_DIM)))
    weights = normal((q_len, heads)) / 8
    query_scale = torch.rand((q_len, heads), generator=gen, device=dev, dtype=torch.float32) + 0.5
    key_scale = torch.rand((blocks, BLOCK_TOKENS), generator=gen, device=dev, dtype=torch.float32) * 1.5 + 0.5
    if qk == "bf16":
        query_scale = key_scale = None
    positions = np.arange(k_len - q_len, k_len, dtype=np.int64)
    slots = table[0, positions // BLOCK_TOKENS].astype(np.int64) * BLOCK_TOKENS + positions % BLOCK_TOKENS
    return dict(query=query, weights=weights, query_scale=query_scale, keys=keys, key_scale=key_scale,
                block_table=torch.from_numpy(table).to(dev), cu_seqlens_q=torch.tensor([0, q_len], dtype=torch.int32,
                                                                                       device=dev),
                seq_lens_k=torch.tensor([k_len], dtype=torch.int32, device=dev),
                slot_mapping=torch.from_numpy(slots).to(dev), positions=torch.from_numpy(positions).to(dev),
                q_len=q_len, k_len=k_len, heads=heads)


def _filled_pool(torch, gen, owners, history, resident, device):
    """Pinned host KV pool of random 656-byte rows for every (owner, position) and the hot
    cache holding positions [0, resident) of each owner, so every hit and every Fetch is
    byte-checkable."""
    pool = torch.empty(owners * history * 656, dtype=torch.uint8, pin_memory=True)
    rows = history * 656
    for o in range(owners):
        pool[o * rows:(o + 1) * rows].copy_(torch.randint(0, 256, (rows,), generator=gen, device=device,
                                                          dtype=torch.uint8))
    hot = torch.empty((owners, resident, 656), dtype=torch.uint8, device=device)
    hot.copy_(pool.view(owners, history, 656)[:, :resident])
    return pool, hot


def mixed_workload(torch, kvip, device, *, seed=2026, decode_ctx=None, history=65536, resident=16384,
                   prefill=((2048, 8192), (1536, 1536)), heads=64, lru=False, fill_pool=False, overlap=True,
                   prefill_after=None, prefill_workgroups=None):
    """config 5 round: decode requests (one row each, contexts `decode_ctx`, default
    32 requests ~U[4096, 65536]) on the resident cache (owner Index rows of `history`
    positions, `resident` hot slots, misses from a pinned host pool) plus prefill chunks
    (q_len, k_len) packed TND-style against a paged index-K cache; every new token (the
    last position of each decode request, the chunks' rows) is ingested into the Index
    storage. lru: the decode requests' victim candidates come from a SlotLRUChains that
    the round commits every step (else fixed candidates 0..2047); fill_pool: random KV
    bytes in the host pool with the hot cache holding each owner's first `resident` rows
    (else the pool is left uninitialised, enough for timing). Returns a SimpleNamespace
    with the bound `round` (a kvip.MixedRound) and its parts; inputs are seeded and already
    resident on the device."""
    from types import SimpleNamespace

    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dev = torch.device(device)
    if decode_ctx is None:
        decode_ctx = rng.integers(4096, history + 1, size=32)
    decode_ctx = np.asarray(decode_ctx, dtype=np.int64)
    nd, npf = len(decode_ctx), len(prefill)
    owners = nd + npf

    def normal(shape):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)

    # Persistent Index storage (fp8 codes with the NaN bit pattern masked out) and KV rows.
    keys = (torch.randint(0, 256, (owners, history, 128), generator=gen, device=dev, dtype=torch.uint8) & 0x77)
    keys = keys.view(torch.float8_e4m3fn)
    scales = torch.rand((owners, history), generator=gen, device=dev) * 1.5 + 0.5
    addresses = (torch.arange(owners * history, device=dev, dtype=torch.int64) * 656).view(owners, history)
    logical = torch.arange(history, device=dev, dtype=torch.int64).repeat(owners, 1)
    if fill_pool:
        pool, hot = _filled_pool(torch, gen, owners, history, resident, dev)
    else:
        pool = torch.empty(owners * history * 656, dtype=torch.uint8, pin_memory=True)
        hot = torch.zeros((owners, resident, 656), dtype=torch.uint8, device=dev)
    valid = torch.ones((owners, resident), dtype=torch.int32, device=dev)
    # Paged index-K cache: the prefill sequences' pages, then one page per 128 decode tokens.
    pf_blocks = [(k + BLOCK_TOKENS - 1) // BLOCK_TOKENS for _, k in prefill]
    dec_blocks = (nd + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    nblocks = sum(pf_blocks) + dec_blocks
    perm = rng.permutation(nblocks).astype(np.int32)
    cache_keys = saturating_fp8(torch, normal((nblocks, BLOCK_TOKENS, INDEX_DIM)))
    cache_scales = torch.rand((nblocks, BLOCK_TOKENS), generator=gen, device=dev) * 1.5 + 0.5
    max_pf_blocks = max(pf_blocks)
    pf_table = np.zeros((npf, max_pf_blocks), np.int32)
    at = 0
    for s, nb in enumerate(pf_blocks):
        pf_table[s, :nb] = perm[at:at + nb]
        at += nb
    dec_pages = perm[at:at + dec_blocks]
    # New tokens: decode request b's token at position ctx_b - 1, then the chunks' rows.
    sources, targets = [], []
    for b, c in enumerate(decode_ctx):
        sources.append(int(dec_pages[b // BLOCK_TOKENS]) * BLOCK_TOKENS + b % BLOCK_TOKENS)
        targets.append(b * history + int(c) - 1)
    for s, (q_len, k_len) in enumerate(prefill):
        pos = np.arange(k_len - q_len, k_len)
        sources += list(pf_table[s, pos // BLOCK_TOKENS].astype(np.int64) * BLOCK_TOKENS + pos % BLOCK_TOKENS)
        targets += list((nd + s) * history + pos)
    # Decode binding on the resident cache.
    rot = kvip.LIFetchBinding(torch, batch=nd, max_context=history, device=dev, heads=heads, rows_per_request=1,
                              qk_dtype="fp8", query_ends=True)
    rot.query.copy_(saturating_fp8(torch, normal(tuple(rot.query.shape))))
    rot.weights.copy_(normal(tuple(rot.weights.shape)) / 8)
    ctx_t = torch.from_numpy(decode_ctx.astype(np.int32)).to(dev)
    rot.seq_lens.copy_(ctx_t)
    rot.query_ends.copy_(ctx_t)
    upd = kvip.ResidentIndexUpdate(torch, overlap=overlap, keys=keys, scales=scales, addresses=addresses,
                                   logical_ids=logical,
                                   row_owners=torch.arange(nd, dtype=torch.int32, device=dev), rotating=rot,
                                   hot_valid=valid, hot_cache=hot, host_pool=pool, resident=resident)
    chains = None
    if lru:
        chains = kvip.SlotLRUChains(torch, nd, resident, dev, slots=upd.lru_slots)
    else:
        upd.set_candidates(torch.arange(2048, dtype=torch.int32, device=dev).repeat(nd, 1))
    # Prefill chunks.
    rows = sum(q for q, _ in prefill)
    pf_query = saturating_fp8(torch, normal((rows, heads, INDEX_DIM)))
    pf_weights = normal((rows, heads)) / 8
    pf_qscale = torch.rand((rows, heads), generator=gen, device=dev) + 0.5
    cu = torch.tensor(np.concatenate([[0], np.cumsum([q for q, _ in prefill])]), dtype=torch.int32, device=dev)
    kl = torch.tensor([k for _, k in prefill], dtype=torch.int32, device=dev)
    table = torch.from_numpy(pf_table).to(dev)
    pidx = kvip.PrefillIndexer(torch, max_rows=rows, max_context=max_pf_blocks * BLOCK_TOKENS, max_sequences=npf,
                               device=dev, heads=heads)
    pidx.bind(pf_query, pf_weights, pf_qscale, cache_keys, cache_scales, cu, kl, table)
    forward = kvip.LIFetch(rot, upd)
    rnd = kvip.MixedRound(torch, decode=forward, prefill=pidx, storage_keys=keys, storage_scales=scales,
                          cache_keys=cache_keys, cache_scales=cache_scales, new_tokens=len(sources), lru=chains,
                          overlap=overlap, prefill_after=prefill_after, prefill_workgroups=prefill_workgroups)
    rnd.sources.copy_(torch.tensor(sources, dtype=torch.int64))
    rnd.targets.copy_(torch.tensor(targets, dtype=torch.int64))
    return SimpleNamespace(round=rnd, rot=rot, update=upd, forward=forward, prefill=pidx, lru=chains, keys=keys,
                           scales=scales,
                           addresses=addresses, logical=logical, hot=hot, valid=valid, pool=pool,
                           cache_keys=cache_keys, cache_scales=cache_scales, pf_query=pf_query, pf_weights=pf_weights,
                           pf_qscale=pf_qscale, cu=cu, kl=kl, table=table, decode_ctx=decode_ctx, chunks=prefill,
                           history=history, resident=resident, sources=sources, targets=targets)


def bind(torch, kvip, wl, *, query_ends=None):
    """LIFetchBinding + ContiguousFetch + LIFetch forward for a workload."""
    heads = int(wl.query.shape[1])
    qk = "fp8" if wl.query.dtype == torch.float8_e4m3fn else "bf16"
    rot = kvip.LIFetchBinding(torch, batch=wl.batch, max_context=wl.max_blocks * BLOCK_TOKENS,
                              device=wl.query.device, heads=heads, rows_per_request=wl.rows_per_request,
                              qk_dtype=qk, weight_dtype=wl.weights.dtype, query_scale=wl.query_scale is not None,
                              query_ends=query_ends is not None)
    rot.query.copy_(wl.query)
    rot.weights.copy_(wl.weights)
    if wl.query_scale is not None:
        rot.query_scale.copy_(wl.query_scale)
    rot.seq_lens.copy_(torch.from_numpy(wl.ctx.astype(np.int32)))
    if query_ends is not None:
        rot.query_ends.copy_(torch.as_tensor(np.asarray(query_ends, np.int32)))
    rot.block_table.copy_(wl.block_table)
    rot.bind_index_cache(wl.keys, wl.key_scale)
    upd = kvip.ContiguousFetch(torch, rot, wl.kv_cache)
    return rot, upd, kvip.LIFetch(rot, upd)


def _bitmap_words(torch, slots, words):
    """int32 [words] membership bitmap of distinct slot ids (device tensor)."""
    acc = torch.zeros(words, dtype=torch.int64, device=slots.device)
    acc.index_add_(0, (slots >> 5).long(), (1 << (slots & 31).long()))
    return ((acc + (1 << 31)) % (1 << 32) - (1 << 31)).to(torch.int32)


def lidu_workload(torch, device, *, seed=2026, batch=16, queries=4, budget=16384, cand=131072, hit=0.8,
                  query_overlap=0.9, num_layers=61, layer_id=7):
    """Inputs of one kvip.lidu call in the reference argument order (config 4
    shape: `batch` MTP requests of `queries` rows, resident budget `budget` of a
    `cand`-token history). Every request owns a pool row holding a random resident set
    of `budget` history tokens; each TopK row takes `hit` of its tokens from the resident
    set, consecutive query rows of a request share `query_overlap` of their tokens, and
    the victims are 2048 random resident slots. Returns (inputs, outputs, call args)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    pool = batch + 1  # + the reserved graph-padding entry
    t2s = torch.full((pool, cand), -1, dtype=torch.int32)
    s2t = torch.full((pool, budget), -1, dtype=torch.int32)
    miss_slots = torch.empty((batch, 2048), dtype=torch.int32)
    topk = torch.empty((batch * queries, 1, 2048), dtype=torch.int32)
    n_hit = int(2048 * hit)
    for b in range(batch):
        resident = torch.randperm(cand, generator=g)[:budget]
        slots = torch.randperm(budget, generator=g)
        t2s[b, resident] = slots.int()
        s2t[b, slots] = resident.int()
        miss_slots[b] = torch.randperm(budget, generator=g)[:2048].int()
        cold = torch.ones(cand, dtype=torch.bool)
        cold[resident] = False
        cold = cold.nonzero().view(-1)
        hits = resident[torch.randperm(budget, generator=g)[:n_hit]]
        misses = cold[torch.randperm(len(cold), generator=g)[:2048 - n_hit]]
        row = torch.cat((hits, misses))
        for q in range(queries):
            if q:
                keep = int(2048 * query_overlap)
                fresh_h = resident[torch.randperm(budget, generator=g)[:2048]]
                fresh_h = fresh_h[~torch.isin(fresh_h, row)][:int((2048 - keep) * hit)]
                fresh_m = cold[torch.randperm(len(cold), generator=g)[:4096]]
                fresh_m = fresh_m[~torch.isin(fresh_m, row)][:2048 - keep - len(fresh_h)]
                row = torch.cat((row[torch.randperm(2048, generator=g)[:keep]], fresh_h, fresh_m))
            topk[b * queries + q, 0] = row[torch.randperm(2048, generator=g)].int()
    blocks = torch.randperm(1 << 20, generator=g)[:batch * (budget // 128)].int().view(batch, -1)
    dev = dict(
        topk=topk, actual_seq_lengths_query=torch.arange(1, batch + 1, dtype=torch.int32) * queries,
        req_pool_entries=torch.arange(batch, dtype=torch.int32), token_to_slot_pool=t2s, slot_to_token_pool=s2t,
        eviction_cursors=torch.zeros(pool, dtype=torch.int32), cache_tokens=torch.full((batch,), budget, dtype=torch.int32),
        candidate_lens=torch.full((batch,), cand, dtype=torch.int32), miss_slots=miss_slots,
        resident_block_table=blocks, logical_seq_lengths=torch.full((batch,), cand + 1, dtype=torch.int32),
        profile_enabled=torch.zeros(1, dtype=torch.int32),
    )
    dev = {k: v.to(device) for k, v in dev.items()}
    dev["miss_slot_bitmap"] = torch.stack([_bitmap_words(torch, dev["miss_slots"][b], 4176) for b in range(batch)])
    cap = batch * 8192
    outs = dict(destination_slots=torch.empty_like(dev["topk"]),
                miss_counts=torch.empty(batch + 1, dtype=torch.int32, device=device),
                indices=torch.empty(cap, dtype=torch.int32, device=device),
                offsets=torch.empty(cap, dtype=torch.int32, device=device),
                output_indices=torch.empty(cap, dtype=torch.int32, device=device),
                resident_seq_lengths=torch.empty(batch, dtype=torch.int32, device=device),
                profiling=torch.zeros((batch, 8, 32), dtype=torch.int64, device=device))
    order = ("topk", "actual_seq_lengths_query", "req_pool_entries", "token_to_slot_pool", "slot_to_token_pool",
             "eviction_cursors", "cache_tokens", "candidate_lens", "miss_slots", "miss_slot_bitmap",
             "resident_block_table", "logical_seq_lengths", "profile_enabled")
    args = [dev[k] for k in order] + list(outs.values()) + [layer_id, num_layers, pool, (cand + 127) // 128]
    return dev, outs, args


def resident_workload(torch, kvip, device, *, seed=2026, batch=16, history=131072, resident=16384, q_rows=1,
                      heads=64, fill_pool=False, prefetch=None, overlap=True):
    """config 4 shape for the resident-cache round: `batch` requests, each owning
    `history` Index rows (fp8 keys ~ random finite codes, scales U(0.5, 2)) and a hot
    cache of `resident` slots holding positions 0..resident-1; every row's KV lives in a
    pinned host pool (random bytes with fill_pool, the hot cache then holding each owner's
    first `resident` rows; else uninitialised, enough for timing); prefetch: a
    ResidentPrefetch for the speculative windowed prefetch. Returns (rotating, update,
    forward)."""
    g = torch.Generator(device=device).manual_seed(seed)
    owners = batch
    keys = (torch.randint(0, 256, (owners, history, 128), generator=g, device=device, dtype=torch.uint8) & 0x77)
    keys = keys.view(torch.float8_e4m3fn)
    scales = torch.rand((owners, history), generator=g, device=device) * 1.5 + 0.5
    addresses = (torch.arange(owners * history, device=device, dtype=torch.int64) * 656).view(owners, history)
    logical = torch.arange(history, device=device, dtype=torch.int64).repeat(owners, 1)
    if fill_pool:
        pool, hot = _filled_pool(torch, g, owners, history, resident, device)
    else:
        pool = torch.empty(owners * history * 656, dtype=torch.uint8, pin_memory=True)
        hot = torch.zeros((owners, resident, 656), dtype=torch.uint8, device=device)
    valid = torch.ones((owners, resident), dtype=torch.int32, device=device)
    rot = kvip.LIFetchBinding(torch, batch=batch, max_context=history, device=device, heads=heads,
                              rows_per_request=q_rows, qk_dtype="fp8", query_ends=True)
    rot.query.copy_(saturating_fp8(torch, torch.randn(rot.query.shape, generator=g, device=device)))
    rot.weights.copy_(torch.randn(rot.weights.shape, generator=g, device=device) / 8)
    rot.seq_lens.fill_(history)
    rot.query_ends.fill_(history)
    upd = kvip.ResidentIndexUpdate(torch, keys=keys, scales=scales, addresses=addresses, logical_ids=logical,
                                   row_owners=torch.arange(batch, dtype=torch.int32, device=device), rotating=rot,
                                   hot_valid=valid, hot_cache=hot, host_pool=pool, resident=resident,
                                   prefetch=prefetch, overlap=overlap)
    return rot, upd, kvip.LIFetch(rot, upd)


def resident_selections(torch, rng, *, steps, batch, q_rows, history, resident, hot_share=0.8, zipf=1.1):
    """TopK rows for `steps` rounds: `hot_share` of every row drawn from the hot positions
    with Zipf(`zipf`) popularity over a fixed random ranking (so consecutive steps revisit
    the same positions), the rest uniform over the cold positions; rows of one request
    share 90 % of their positions. Returns int32 [steps, batch * q_rows, 2048]."""
    out = np.full((steps, batch * q_rows, 2048), -1, np.int32)
    rank = rng.permutation(resident)
    weights = 1.0 / np.arange(1, resident + 1) ** zipf
    weights /= weights.sum()
    n_hot = int(2048 * hot_share)
    for s in range(steps):
        for b in range(batch):
            hot = rank[rng.choice(resident, n_hot, replace=False, p=weights)]
            cold = rng.choice(np.arange(resident, history), 2048 - n_hot, replace=False)
            base = np.concatenate([hot, cold])
            for q in range(q_rows):
                row = base.copy()
                if q:
                    swap = rng.random(2048) < 0.1
                    fresh = rng.choice(np.arange(resident, history), int(swap.sum()) * 2, replace=False)
                    fresh = np.setdiff1d(fresh, base)[:int(swap.sum())]
                    row[np.nonzero(swap)[0][:len(fresh)]] = fresh
                out[s, b * q_rows + q] = rng.permutation(row)
    return out
