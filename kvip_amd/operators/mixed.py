"""One continuous-batching round over decode requests and packed prefill chunks.

The reference's vLLM selector runs a mixed batch as: Index ingest of the round's new tokens
(python/kvip/adapters/vllm/selector.py:102-106 -> index_import.py:17-56), the fused LIFetch
forward for the decode rows (:110-112) and the native prefill indexer for each prefill
chunk (:126-154). `MixedRound` enqueues the same three stages on the current stream with
buffers bound once, so the whole round is one hipGraph (config 5):

  1. one list-mode `kvip_hip_ingest_index` launch copies every new token's index-K row and
     scale from the paged cache (`sources`: cache row = block * 128 + offset) to its Index
     storage row (`targets`: owner * history + position);
  2. the decode forward (`kvip_amd.LIFetch` over a `ResidentIndexUpdate`, or a
     `ContiguousFetch`): LI over the owners' Index rows, TopK, resolver, Fetch, Index update
     and outputs;
  3. with `lru` (a SlotLRUChains whose `slots` are the resident update's candidates), one
     launch committing every decode request's selected slots, attached to the resident
     update so that it runs right after the Index update (beside the Fetch), so the next
     round's victim candidates follow the cache's own recency, as the reference's selector
     commits each request's SlotLRU after a step (python/kvip/cache/lru.py:96-118);
  4. the prefill indexer bound with `PrefillIndexer.bind`: LI over the paged cache for the
     packed chunks (cumulative query lengths) and TopK-2048 per row.

The prefill stage reads only the paged cache and its own buffers, so it runs on a second
stream joined at the round's end (`overlap=True`, the default), forked at the point
`prefill_after` names: "start" (default: at the round's start, beside everything), "scoring"
(after the decode's scoring is enqueued) or "resolve" (resident decode: after its scoring,
TopK and resolve, so that the prefill overlaps only the PCIe-bound Fetch, the Index update
and the LRU commit). On MI355X at config 5 the three measured 304, 310 and 312-320
us per round: two prefill workgroups fill a CU's LDS, so the later fork points leave the
short decode kernels alone but serialise the prefill behind them. The fork and join are
events, so the round stays one capturable sequence on the caller's stream.

The caller fills the per-round inputs in place before a launch or replay: decode Q /
weights / lengths, the prefill buffers it bound, and `sources` / `targets` of the new
tokens. Device errors land in the status words of the three stages.
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi

INDEX_DIM = 128


class MixedRound:
    def __init__(self, torch, *, decode, prefill, storage_keys, storage_scales, cache_keys, cache_scales,
                 new_tokens, status=None, lru=None, overlap=True, prefill_after=None, prefill_workgroups=None):
        """decode: a LIFetch forward; prefill: a PrefillIndexer after `bind(...)`;
        storage_keys [owners, history, 128] (fp8 or uint8) and storage_scales
        [owners, history] float32: the persistent Index rows; cache_keys
        [blocks, 128, 128] and cache_scales [blocks, 128]: the paged index-K cache the new
        tokens are read from; new_tokens: rows ingested per round."""
        if getattr(prefill, "_args", None) is None:
            raise ValueError("bind the prefill indexer before building the round")
        if storage_keys.dim() != 3 or storage_keys.shape[2] != INDEX_DIM or storage_keys.element_size() != 1:
            raise ValueError("Index storage keys must be 1-byte [owners, history, 128]")
        if not storage_keys.is_contiguous() or storage_scales.dtype != torch.float32 or not storage_scales.is_contiguous():
            raise ValueError("Index storage must be contiguous with float32 scales")
        if tuple(storage_scales.shape) != tuple(storage_keys.shape[:2]):
            raise ValueError("Index storage scales must be [owners, history]")
        if cache_keys.dim() != 3 or tuple(cache_keys.shape[1:]) != (128, INDEX_DIM) or cache_keys.element_size() != 1:
            raise ValueError("paged index-K cache must be 1-byte [blocks, 128, 128]")
        if not cache_keys.is_contiguous() or cache_scales.dtype != torch.float32 or not cache_scales.is_contiguous():
            raise ValueError("paged index-K cache and its scales must be contiguous (scales float32)")
        if tuple(cache_scales.shape) != tuple(cache_keys.shape[:2]):
            raise ValueError("paged key scales must be [blocks, 128]")
        if new_tokens < 1:
            raise ValueError("a round ingests at least one new token")
        dev = storage_keys.device
        self.torch, self.decode, self.prefill, self.device = torch, decode, prefill, dev
        self.storage_keys, self.storage_scales = storage_keys, storage_scales
        self.cache_keys, self.cache_scales = cache_keys, cache_scales
        self.sources = torch.zeros(new_tokens, dtype=torch.int64, device=dev)
        self.targets = torch.zeros(new_tokens, dtype=torch.int64, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev) if status is None else status
        p = abi.ptr
        self.ingest_args = abi.IngestArgs(
            source_keys=p(cache_keys), source_scales=p(cache_scales), target_keys=p(storage_keys),
            target_scales=p(storage_scales), sources=p(self.sources), targets=p(self.targets),
            status=p(self.status), source_rows=cache_keys.shape[0] * 128,
            target_rows=storage_keys.shape[0] * storage_keys.shape[1], count=new_tokens, target_base=0,
            mode=abi.INGEST_LIST)
        self.library = abi.load_library()
        self.lru = lru
        if lru is not None:
            if not getattr(decode, "resident", False):
                raise ValueError("the LRU chains must feed a resident decode update's candidates")
            # Committed by the decode round itself, right after its Index update.
            decode.update.attach_lru(lru)
        self.overlap = overlap
        resident = getattr(decode, "resident", False)
        if prefill_after is None:
            prefill_after = "start"
        if prefill_after not in ("start", "scoring", "resolve"):
            raise ValueError(f"prefill_after must be 'start', 'scoring' or 'resolve' (got {prefill_after!r})")
        if prefill_after == "resolve" and not resident:
            raise ValueError("prefill_after='resolve' needs a resident decode update")
        if prefill_after != "start" and not hasattr(decode, "after_scoring"):
            raise ValueError("the decode forward has no stage hooks: use prefill_after='start'")
        self.prefill_after = prefill_after
        # The prefill's scoring grid beside the decode: twice the CU count (two prefill
        # workgroups fill a CU's LDS), so that CUs whose workgroups run out of work units go
        # to the decode kernels instead of to queued prefill workgroups; 0 = one workgroup
        # per unit. In sequence (overlap=False) the prefill runs alone on its full grid.
        if prefill_workgroups is None:
            prefill_workgroups = 2 * torch.cuda.get_device_properties(dev).multi_processor_count if overlap else 0
        if int(prefill_workgroups) < 0:
            raise ValueError("prefill_workgroups must be >= 0")
        self.prefill_workgroups = int(prefill_workgroups)
        self._forks = 0
        if overlap:
            # The prefill branch: its own stream (default priority) and the fork/join events.
            self.side = torch.cuda.Stream(device=dev)
            self.forked, self.joined = torch.cuda.Event(), torch.cuda.Event()

    def ingest(self):
        abi.check(self.library.kvip_hip_ingest_index(ctypes.byref(self.ingest_args),
                                                     abi.stream_handle(self.torch, self.device)), "mixed ingest")

    def _fork(self, main):
        """Enqueue the prefill stage on the second stream, after what `main` holds so far."""
        self.forked.record(main)
        self.side.wait_event(self.forked)
        with self.torch.cuda.stream(self.side):
            self.prefill.score(workgroups=self.prefill_workgroups)
            self.prefill.select()
        self.joined.record(self.side)
        self._forks += 1

    def __call__(self):
        torch = self.torch
        if not self.overlap:
            self.ingest()
            self.decode()
            self.prefill.score(workgroups=self.prefill_workgroups)
            return self.prefill.select()
        main = torch.cuda.current_stream(self.device)
        self._forks = 0
        if self.prefill_after == "start":
            self._fork(main)
            self.ingest()
            self.decode()
        else:
            owner = self.decode.update if self.prefill_after == "resolve" else self.decode
            name = "after_resolve" if self.prefill_after == "resolve" else "after_scoring"
            setattr(owner, name, self._fork)
            try:
                self.ingest()
                self.decode()
            finally:
                setattr(owner, name, None)
        if self._forks != 1:
            raise RuntimeError(f"mixed round: the prefill stage was enqueued {self._forks} times")
        torch.cuda.current_stream(self.device).wait_event(self.joined)
        return self.prefill.topk[:self.prefill._rows]
