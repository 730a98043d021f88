"""Import vLLM paged Index rows into persistent LIFetch storage on the device.

Same class and methods as the reference (python/kvip/adapters/vllm/index_import.py:
6-52); the row copies run as `kvip_hip_ingest_index` launches instead of torch
index_select / index_copy_ pairs.
"""
from __future__ import annotations

import ctypes

from kvip_amd.cache.index_storage import IndexCacheStorage as _Storage
from kvip_amd.runtime import abi


class VllmIndexCacheStorage(_Storage):
    def _sources(self, cache):
        keys, scales = cache
        if keys.element_size() != 1 or keys.shape[-1] != 128 or scales.dtype != self.torch.float32:
            raise ValueError("LIFetch Index import requires C8 keys and float32 scales")
        source_keys = keys.view(self.torch.uint8).view(-1, 128)
        source_scales = scales.view(-1)
        if source_keys.shape[0] != source_scales.numel():
            raise ValueError("Paged Index key and scale capacities differ")
        if source_keys.device != self.device or source_scales.device != self.device:
            raise ValueError("Paged Index cache and storage must share a device")
        return source_keys, source_scales

    def _ingest(self, source_keys, source_scales, **fields):
        if self.device.type != "cuda":
            raise ValueError("Index ingestion needs GPU tensors (kvip_amd has no CPU path)")
        lib = abi.load_library()
        args = abi.IngestArgs(
            source_keys=abi.ptr(source_keys), source_scales=abi.ptr(source_scales),
            target_keys=abi.ptr(self.keys), target_scales=abi.ptr(self.scales), status=abi.ptr(self.status),
            source_rows=source_keys.shape[0], target_rows=self.keys.shape[0] * self.history, **fields)
        abi.check(lib.kvip_hip_ingest_index(ctypes.byref(args), abi.stream_handle(self.torch, self.device)),
                  "ingest_index")

    def ingest_prefill(self, cache, metadata, plans, positions):
        """Eager prefill (:18-37): a new owner with a restored prefix imports tokens
        [0, plan.start) once through its block table, then the plan's current tokens
        move from slot_mapping[begin:stop] to positions[begin:stop]."""
        source_keys, source_scales = self._sources(cache)
        torch = self.torch
        for row, plan in enumerate(plans):
            owner = plan.owner
            if self.requests.get(owner) != plan.request:
                raise RuntimeError("Index owner must be prepared before ingestion")
            base = owner * self.history
            if owner not in self.imported and plan.start:
                table = metadata.block_table[row].to(torch.int32).contiguous()
                self._ingest(source_keys, source_scales, mode=abi.INGEST_PREFIX, count=plan.start,
                             block_table=abi.ptr(table), block_size=metadata.block_size, target_base=base)
            self.imported.add(owner)
            sources = metadata.slot_mapping[plan.begin:plan.stop].to(torch.int64).contiguous()
            targets = positions[plan.begin:plan.stop].to(torch.int64).contiguous()
            self._ingest(source_keys, source_scales, mode=abi.INGEST_LIST, count=sources.numel(),
                         sources=abi.ptr(sources), targets=abi.ptr(targets), target_base=base)

    def ingest_decode(self, cache, metadata, inputs, row_owners):
        """Fixed-shape graph writes (:39-52): every packed row moves one index-K row to
        (owner, query_end - 1); padding rows write distinct positions of reserved owner 0."""
        source_keys, source_scales = self._sources(cache)
        slots = metadata.slot_mapping
        if slots.dtype != self.torch.int64 or not slots.is_contiguous() or row_owners.dtype != self.torch.int32:
            raise ValueError("decode ingest needs int64 slot_mapping and int32 row owners")
        self._ingest(source_keys, source_scales, mode=abi.INGEST_DECODE, count=inputs.query_ends.numel(),
                     query_ends=abi.ptr(inputs.query_ends), gather_indices=abi.ptr(inputs.gather_indices),
                     slot_mapping=abi.ptr(slots), slot_count=slots.numel(), row_owners=abi.ptr(row_owners),
                     queries_per_request=4, history=self.history)


# Public name kept by the reference for the adapter subclass.
IndexCacheStorage = VllmIndexCacheStorage
