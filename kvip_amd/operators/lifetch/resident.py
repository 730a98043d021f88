"""Resident-cache `update` argument of ``kvip_amd.LIFetch``: the hot/cold LIFetch round.

`ResidentIndexUpdate` mirrors the reference's DirectIndexUpdate
(python/kvip/operators/lifetch/index_update.py:28-102): it binds the stable per-owner
Index storage (keys [owners, history, 128] fp8, scales [owners, history] float32, KV
addresses and logical ids [owners, history] int64), the request -> owner rows and the
service outputs (logical and slot TopK, int32 [2, rows, 1, 2048]). Next to them it binds
what the reference keeps behind KVAF: the hot KV cache [owners, hot_stride, row_bytes]
(position p < resident of an owner is hot slot p) and the host KV pool, a
device-accessible (pinned) host tensor in which `addresses` are byte offsets. With
`query_inputs` (a vLLM-adapter QueryInputs, four query rows per request) the outputs are
published in token order like the reference's (index_update.py:18-21, 85-99): output row
t holds the query row unpack_indices[t] when output_valid[t], else -1 throughout. With
`tail_bounds` ([batch, 2] int32 {begin, end}, the reference binding's tail_bounds,
binding.py:150) positions [begin, end) of each request are its ABC tail: never hot hits,
the first T = hot_stride - resident of them resolved to ring slot resident + p % T of the
hot cache without a Fetch (the hot cache then holds resident + T rows per owner, T a
multiple of 128 and at least 384).

The forward enqueues, on the current stream and without host synchronisation: the
owner block table, LI scoring of the owners' Index rows, TopK-2048 per query row, and the
round of kvip_hip_resident_round (init, resolve, Fetch from the host pool, Index update,
residency). With `prefetch` (a ResidentPrefetch) the forward also runs the speculative
windowed prefetch (the reference's FastService, op_kernel/prefetch.h:578-832) on a second
stream while the final TopK runs: the prefix TopK of the hot positions gives each query
row a threshold, and the candidates and cold positions above it are fetched ahead into
LRU candidate slots; the final round then resolves selected prefetched tokens to those
slots and fetches only the rest. Outputs (logical ids, and the KV bytes behind every slot)
are those of the round without prefetch. Per-step inputs are `rotating.lru_slots` ([batch, 2048] victim candidates,
oldest first, e.g. ``SlotLRU.slots``) plus the query buffers of the binding. Device
errors land in `status` ([batch] int32, KVIP_RESIDENT_ERR_* bits).
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi
from kvip_amd.operators.lifetch.binding import BLOCK_TOKENS, INDEX_DIM, TOPK

LRU_SLOTS = abi.RESIDENT_LRU_SLOTS


class ResidentPrefetch:
    """Budgets of the speculative windowed prefetch (python/kvip/operators/lifetch/
    geometry.py:4-13 prefetch_budget, :55-61 trigger_tokens): `windows` windows (the first
    takes the victim candidates, the others the cold range split at the 128-aligned trigger
    boundaries), at most `window_limit` fetches per window (default prefetch_limit //
    windows) and `prefetch_limit` per request and round."""

    def __init__(self, windows=8, prefetch_limit=512, window_limit=None, windowed=False):
        """windowed: score the Index window by window and make each window's prefetch
        decisions and host copies on other streams as soon as it is scored (fp8 scoring with
        one query row per request; same results). Off by default: on MI355X the scoring of
        a C4 round split into 8 launches takes ~140 us against ~73 us in one, and the
        decision kernels wait for CUs behind each scoring launch, so the round is slower
        than scoring first and prefetching after."""
        if type(windows) is not int or not 1 <= windows <= 32:
            raise ValueError("Prefetch requires 1..32 windows")
        if window_limit is None:
            window_limit = max(1, prefetch_limit // windows)
        if not 0 <= prefetch_limit <= LRU_SLOTS or not 1 <= window_limit <= 480:
            raise ValueError("Invalid prefetch budgets: total must be 0..2048 and window 1..480")
        self.windows, self.prefetch_limit, self.window_limit = windows, int(prefetch_limit), int(window_limit)
        self.windowed = bool(windowed)


class ResidentIndexUpdate:
    def __init__(self, torch, *, keys, scales, addresses, logical_ids, row_owners, rotating, hot_valid, hot_cache,
                 host_pool, resident, status=None, outputs=None, used=0, query_inputs=None, tail_bounds=None,
                 prefetch=None, overlap=True):
        """overlap: run each round's Fetch of the misses beside its Index update (and the
        attached LRU commit) on a second stream after the resolve, joined before the round
        ends (`finish()`); False keeps the three stages on the caller's stream. Results are
        the same either way."""
        self.torch, self.rotating, self.device = torch, rotating, rotating.device
        if keys.dim() != 3 or keys.shape[2] != INDEX_DIM or keys.dtype != torch.float8_e4m3fn or not keys.is_contiguous():
            raise ValueError("Index keys must be contiguous float8_e4m3fn [owners, history, 128]")
        owners, history = int(keys.shape[0]), int(keys.shape[1])
        if history % BLOCK_TOKENS:
            raise ValueError("Index history must be a multiple of 128 positions")
        for name, t, dtype in (("scales", scales, torch.float32), ("addresses", addresses, torch.int64),
                               ("logical_ids", logical_ids, torch.int64)):
            if tuple(t.shape) != (owners, history) or t.dtype != dtype or not t.is_contiguous():
                raise ValueError(f"Index {name} must be contiguous {dtype} [owners, history]")
        if row_owners.dtype != torch.int32 or tuple(row_owners.shape) != (rotating.batch,):
            raise ValueError("row_owners must be int32 [batch]")
        if not abi.RESIDENT_LRU_SLOTS <= resident <= min(history, abi.RESIDENT_MAX_RESIDENT):
            raise ValueError(f"resident must be in 2048..min(history, {abi.RESIDENT_MAX_RESIDENT})")
        if tuple(hot_valid.shape) != (owners, resident) or hot_valid.dtype != torch.int32:
            raise ValueError("hot_valid must be int32 [owners, resident]")
        if (hot_cache.dim() != 3 or hot_cache.shape[0] != owners or hot_cache.shape[1] < resident or
                hot_cache.dtype != torch.uint8 or not hot_cache.is_contiguous() or hot_cache.shape[2] % 16):
            raise ValueError("hot cache must be contiguous uint8 [owners, >= resident, row_bytes % 16 == 0]")
        if host_pool.dtype != torch.uint8 or host_pool.device.type != "cpu" or not host_pool.is_pinned():
            raise ValueError("host pool must be a pinned uint8 CPU tensor (device-mapped host memory)")
        if rotating.rows_per_request > abi.RESIDENT_MAX_QUERIES or rotating.qk_name != "fp8":
            raise ValueError("resident LIFetch supports fp8 Index keys and up to 4 query rows per request")
        if rotating.max_blocks * BLOCK_TOKENS < history:
            raise ValueError("LIFetch binding max_context must cover the Index history")
        if not 0 <= used <= LRU_SLOTS:
            raise ValueError("used must be in 0..2048")
        if query_inputs is not None and (rotating.rows_per_request != 4 or query_inputs.batch != rotating.batch or
                                         query_inputs.device != rotating.device):
            raise ValueError("token-order outputs need the binding's batch, four query rows and device")
        dev = self.device
        if tail_bounds is not None:
            ring = int(hot_cache.shape[1]) - resident
            if (tail_bounds.dtype != torch.int32 or tuple(tail_bounds.shape) != (rotating.batch, 2) or
                    not tail_bounds.is_contiguous() or tail_bounds.device != dev):
                raise ValueError(f"tail_bounds must be contiguous int32 [{rotating.batch}, 2] on {dev}")
            if ring < 384 or ring % 128:
                raise ValueError("ABC tail bounds need hot-cache ring slots after the hot ones: hot_cache.shape[1] "
                                 "- resident must be a multiple of 128 and at least 384")
        self.tail_bounds = tail_bounds
        if prefetch is not None:
            if not isinstance(prefetch, ResidentPrefetch):
                raise ValueError("prefetch must be a ResidentPrefetch")
            if resident % BLOCK_TOKENS or (history - resident) // BLOCK_TOKENS <= prefetch.windows:
                raise ValueError("prefetch needs a 128-aligned resident range and more cold 128-token tiles "
                                 "than windows")
        self.prefetch = prefetch
        if any(t.device != dev for t in (keys, scales, addresses, logical_ids, row_owners, hot_valid, hot_cache)):
            raise ValueError("Index storage, hot cache and the LIFetch binding must share one device")
        self.keys, self.scales, self.addresses, self.logical_ids = keys, scales, addresses, logical_ids
        self.row_owners, self.hot_valid, self.hot_cache, self.host_pool = row_owners, hot_valid, hot_cache, host_pool
        self.query_inputs = query_inputs
        self.owners, self.history, self.resident, self.used = owners, history, resident, used
        rows, q = rotating.rows, rotating.rows_per_request
        self.status = torch.zeros(rotating.batch, dtype=torch.int32, device=dev) if status is None else status
        if outputs is None:
            outputs = torch.full((2, rows, 1, TOPK), -1, dtype=torch.int32, device=dev)
        if tuple(outputs.shape) != (2, rows, 1, TOPK) or outputs.dtype != torch.int32 or not outputs.is_contiguous():
            raise ValueError("Service outputs must be contiguous int32 [2, rows, 1, 2048]")
        self.outputs = outputs
        self.logical_output, self.slot_output = outputs.unbind(0)
        b = rotating.batch
        # Round state (the reference's rotation scratch, workspace.py:9-31).
        self.lru_slots = rotating.lru_slots = torch.full((b, LRU_SLOTS), -1, dtype=torch.int32, device=dev)
        self.reserved_hot = torch.full((b, resident), -1, dtype=torch.int32, device=dev)
        nchg = LRU_SLOTS + q * TOPK
        self.changes = torch.full((b, nchg), -1, dtype=torch.int32, device=dev)
        self.change_slots = torch.full((b, nchg), -1, dtype=torch.int32, device=dev)
        self.miss_counts = torch.zeros((b, 5), dtype=torch.int32, device=dev)
        self.fetch_sources = torch.zeros((b, q * TOPK), dtype=torch.int64, device=dev)
        self.fetch_slots = torch.zeros((b, q * TOPK), dtype=torch.int32, device=dev)
        self.fetch_positions = torch.zeros((b, q * TOPK), dtype=torch.int32, device=dev)
        # Prefetch records: the token of every prefetch ordinal and the count per request.
        self.prefetch_tokens = self.prefetch_counts = None
        if prefetch is not None:
            self.prefetch_tokens = torch.full((b, LRU_SLOTS), -1, dtype=torch.int32, device=dev)
            self.prefetch_counts = torch.zeros(b, dtype=torch.int32, device=dev)
        lib = abi.load_library()
        nbytes = int(lib.kvip_hip_resident_workspace_bytes(b, history))
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        # LI reads the owners' Index rows as 128-position blocks.
        rotating.bind_index_cache(keys.view(owners * history // BLOCK_TOKENS, BLOCK_TOKENS, INDEX_DIM),
                                  scales.view(owners * history // BLOCK_TOKENS, BLOCK_TOKENS))
        if rotating.query_ends is None:
            rotating.seq_lens.fill_(history)
        self.args = self.resident_args()
        self._ref = ctypes.byref(self.args)
        self.library = lib
        abi.check(lib.kvip_hip_resident_prepare(self._ref, abi.stream_handle(torch, dev)), "resident workspace")
        self.lru = self.commit_rows = None
        # Called with the launch stream right after each round's resolve is enqueued (the
        # point from which a caller may fork work that should not compete with the scoring,
        # TopK and resolve for compute units); None: nothing.
        self.after_resolve = None
        self.overlap = bool(overlap)
        if self.overlap:
            # The Index-update branch: its own stream (default priority), forked after the
            # resolve and joined after the Fetch.
            self.side = torch.cuda.Stream(device=dev)
            self.resolved, self.updated = torch.cuda.Event(), torch.cuda.Event()

    def attach_lru(self, chains):
        """Commit `chains` (a SlotLRUChains with one chain per request whose `slots` alias
        this update's lru_slots) with each round's selected slots right after the round's
        Index update, so the next round's victim candidates follow the cache's recency (the
        reference's selector commits each request's SlotLRU after a step,
        python/kvip/cache/lru.py:96-118). With overlap the commit runs on the update branch,
        beside the Fetch."""
        if chains.slots.data_ptr() != self.lru_slots.data_ptr():
            raise ValueError("the LRU chains must feed this update's candidates (slots aliasing its lru_slots)")
        if chains.chains != self.rotating.batch:
            raise ValueError(f"{chains.chains} LRU chains for {self.rotating.batch} requests")
        self.lru = chains
        self.commit_rows = self.slot_output.view(self.rotating.batch, -1)

    def finish(self, copies_done=None):
        """The round after its TopK (and prefetch): resolve, then the Fetch of the misses and
        the Index update (+ the attached LRU commit), enqueued on the current stream; with
        overlap the update branch runs on the second stream and is joined before return.
        copies_done: the event of the last prefetch copy of a windowed prefetch, still
        running on its own stream. The resolve needs only the prefetch decisions, but the
        copies read what the Index update and the LRU commit rewrite (each prefetched
        token's host address in `addresses`, its candidate slot in `lru_slots`) and write
        slots the final misses may take, so the Fetch of the misses, the Index update and
        the LRU commit all wait for it. Capturable: no allocation, synchronisation or
        read-back."""
        torch, lib = self.torch, self.library
        main = torch.cuda.current_stream(self.device)
        if not self.overlap:
            if copies_done is None and self.after_resolve is None:
                abi.check(lib.kvip_hip_resident_finish(self._ref, main.cuda_stream), "resident round")
            else:
                abi.check(lib.kvip_hip_resident_resolve(self._ref, main.cuda_stream), "resident resolve")
                if self.after_resolve is not None:
                    self.after_resolve(main)
                if copies_done is not None:
                    main.wait_event(copies_done)  # before the Fetch, the update and the LRU commit
                abi.check(lib.kvip_hip_resident_fetch(self._ref, main.cuda_stream), "resident Fetch")
                abi.check(lib.kvip_hip_resident_update(self._ref, main.cuda_stream), "resident Index update")
            if self.lru is not None:
                self.lru.commit(self.commit_rows)
            return
        abi.check(lib.kvip_hip_resident_resolve(self._ref, main.cuda_stream), "resident resolve")
        if self.after_resolve is not None:
            self.after_resolve(main)
        self.resolved.record(main)
        self.side.wait_event(self.resolved)
        if copies_done is not None:
            self.side.wait_event(copies_done)
        abi.check(lib.kvip_hip_resident_update(self._ref, self.side.cuda_stream), "resident Index update")
        if self.lru is not None:
            with torch.cuda.stream(self.side):
                self.lru.commit(self.commit_rows)
        self.updated.record(self.side)
        if copies_done is not None:
            main.wait_event(copies_done)
        abi.check(lib.kvip_hip_resident_fetch(self._ref, main.cuda_stream), "resident Fetch")
        main.wait_event(self.updated)

    def round(self):
        """kvip_hip_resident_round on the current stream (initialisation, then `finish()`),
        for callers that produce the TopK rows themselves."""
        abi.check(self.library.kvip_hip_resident_begin(self._ref, abi.stream_handle(self.torch, self.device)),
                  "resident round")
        self.finish()

    def set_candidates(self, lru_slots):
        """Victim candidates for the next step ([batch, 2048] int32, oldest first)."""
        self.lru_slots.copy_(lru_slots)

    def resident_args(self):
        p = abi.ptr
        r = self.rotating
        return abi.ResidentArgs(
            topk=p(r.topk), row_owners=p(self.row_owners), lru_slots=p(self.lru_slots),
            reserved_hot=p(self.reserved_hot), hot_valid=p(self.hot_valid), index_keys=p(self.keys),
            index_scales=p(self.scales), addresses=p(self.addresses), logical_ids=p(self.logical_ids),
            host_pool=p(self.host_pool), hot_cache=p(self.hot_cache), logical_output=p(self.logical_output),
            slot_output=p(self.slot_output), changes=p(self.changes), change_slots=p(self.change_slots),
            miss_counts=p(self.miss_counts), fetch_sources=p(self.fetch_sources), fetch_slots=p(self.fetch_slots),
            fetch_positions=p(self.fetch_positions), status=p(self.status), workspace=p(self.workspace),
            host_pool_bytes=self.host_pool.numel(), batch=r.batch, rows_per_request=r.rows_per_request,
            owners=self.owners, history=self.history, resident=self.resident, hot_stride=int(self.hot_cache.shape[1]),
            row_bytes=int(self.hot_cache.shape[2]), used=self.used,
            unpack_indices=p(self.query_inputs.unpack_indices) if self.query_inputs is not None else 0,
            output_valid=p(self.query_inputs.output_valid) if self.query_inputs is not None else 0,
            tail_bounds=p(self.tail_bounds), prefetch_tokens=p(self.prefetch_tokens),
            prefetch_counts=p(self.prefetch_counts),
        )


class ResidentPrefix:
    """Resident TopK of a scored step and its hit bits (what the reference's speculative
    prefetch reads; ProcessResidentTopK + SaveResident, op_kernel/indexer/
    indexer_vector.h:100-105, :162-234): `prefix_topk` [rows, 2048] = TopK-2048 of positions
    [0, resident), `thresholds` [rows] (uint16 keys in int16 storage) = the smallest key of
    a full prefix selection, `victim_hits` [rows, 64] bit i = LRU candidate i scores above
    the threshold, `cold_hits` [rows, words] bit j = position resident + j does. Call after
    scoring (``LIFetch.score()``) and before the next one."""

    def __init__(self, torch, rotating, lru_slots, resident):
        if not 1 <= resident <= rotating.key_stride:
            raise ValueError("resident must be in 1..key_stride")
        if lru_slots.dtype != torch.int32 or tuple(lru_slots.shape) != (rotating.batch, LRU_SLOTS):
            raise ValueError("lru_slots must be int32 [batch, 2048]")
        dev = rotating.device
        self.torch, self.rotating, self.resident, self.lru_slots = torch, rotating, resident, lru_slots
        rows = rotating.rows
        self.cold_words = (rotating.key_stride - resident + 31) // 32
        self.prefix_topk = torch.full((rows, TOPK), -1, dtype=torch.int32, device=dev)
        self.thresholds = torch.zeros(rows, dtype=torch.int16, device=dev)
        self.victim_hits = torch.zeros((rows, TOPK // 32), dtype=torch.int32, device=dev)
        self.cold_hits = torch.zeros((rows, max(self.cold_words, 1)), dtype=torch.int32, device=dev)
        p = abi.ptr
        r = rotating
        self.topk_args = abi.TopkArgs(score_keys=p(r.score_keys), histogram=0, segments=0, seq_lens=p(r.seq_lens),
                                      query_ends=p(r.query_ends), topk=p(self.prefix_topk), status=p(r.status),
                                      batch=r.batch, rows_per_request=r.rows_per_request, key_stride=r.key_stride,
                                      limit=resident)
        self.args = abi.PrefixClassifyArgs(
            score_keys=p(r.score_keys), prefix_topk=p(self.prefix_topk), seq_lens=p(r.seq_lens),
            query_ends=p(r.query_ends), lru_slots=p(lru_slots), thresholds=p(self.thresholds),
            victim_hits=p(self.victim_hits), cold_hits=p(self.cold_hits), batch=r.batch,
            rows_per_request=r.rows_per_request, key_stride=r.key_stride, resident=resident,
            cold_words=self.cold_words)
        self.library = abi.load_library()

    def __call__(self):
        abi.check(self.library.kvip_hip_resident_prefix(ctypes.byref(self.topk_args), ctypes.byref(self.args),
                                                        abi.stream_handle(self.torch, self.rotating.device)),
                  "resident prefix")
