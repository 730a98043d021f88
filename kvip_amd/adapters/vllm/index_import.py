"""vLLM paged index-K rows into the persistent Index storage, on the device.

Interface of the reference's VllmIndexCacheStorage (python/kvip/adapters/vllm/
index_import.py:6-52): `ingest_prefill(cache, metadata, plans, positions)` and
`ingest_decode(cache, metadata, inputs, row_owners)`, with `cache` = (keys, scales) of
vLLM's indexer cache, rows addressed as block * block_size + offset.

Every copy is a `kvip_hip_ingest_index` launch (128 key bytes + one fp32 scale per row):
  prefill  an owner whose request arrives with a restored prefix reads positions
           [0, start) once through its block table (prefix mode); then the step's new
           tokens of every plan move together in one list launch (source = the token's
           slot_mapping entry, target = owner * history + its position);
  decode   one launch over the fixed [batch * 4] packed rows: live rows go to
           (owner, query_end - 1), padding rows to distinct positions of owner 0.
"""
from __future__ import annotations

import ctypes

import numpy as np

from kvip_amd.cache.index_storage import IndexCacheStorage
from kvip_amd.runtime import abi

INDEX_DIM = 128


class VllmIndexCacheStorage(IndexCacheStorage):
    def _paged_rows(self, cache):
        """(keys [rows, 128] uint8, scales [rows] float32) flat views of the paged cache."""
        torch = self.torch
        keys, scales = cache
        if keys.element_size() != 1 or keys.shape[-1] != INDEX_DIM:
            raise ValueError(f"paged index-K must hold 1-byte rows of {INDEX_DIM} (got {keys.dtype}, "
                             f"{tuple(keys.shape)})")
        if scales.dtype != torch.float32:
            raise ValueError(f"paged index-K scales must be float32 (got {scales.dtype})")
        flat_keys, flat_scales = keys.view(torch.uint8).reshape(-1, INDEX_DIM), scales.reshape(-1)
        if flat_keys.shape[0] != flat_scales.shape[0]:
            raise ValueError(f"paged cache holds {flat_keys.shape[0]} key rows but {flat_scales.shape[0]} scales")
        if flat_keys.device != self.device or flat_scales.device != self.device:
            raise ValueError("paged index-K cache and Index storage live on different devices")
        return flat_keys, flat_scales

    def _launch(self, rows, **fields):
        if self.device.type != "cuda":
            raise ValueError("Index ingestion runs on the GPU only (kvip_amd has no CPU path)")
        keys, scales = rows
        args = abi.IngestArgs(source_keys=abi.ptr(keys), source_scales=abi.ptr(scales),
                              target_keys=abi.ptr(self.keys), target_scales=abi.ptr(self.scales),
                              status=abi.ptr(self.status), source_rows=keys.shape[0],
                              target_rows=self.owners * self.history, **fields)
        abi.check(abi.load_library().kvip_hip_ingest_index(ctypes.byref(args),
                                                           abi.stream_handle(self.torch, self.device)),
                  "kvip_hip_ingest_index")

    def ingest_prefill(self, cache, metadata, plans, positions):
        """Eager step: restored prefixes of newly held owners once, then every plan's
        tokens [begin, stop) of the step (slot_mapping -> positions) in one launch."""
        torch = self.torch
        rows = self._paged_rows(cache)
        plans = list(plans)
        spans, bases = [], []
        for row, plan in enumerate(plans):
            rec = self.records.get(int(plan.owner))
            if rec is None or rec.request != plan.request:
                raise RuntimeError(f"owner {plan.owner} was not prepared for request {plan.request!r} "
                                   "before its Index ingestion")
            if not rec.prefix_imported and plan.start:
                table = metadata.block_table[row].to(torch.int32).contiguous()
                self._launch(rows, mode=abi.INGEST_PREFIX, count=int(plan.start), block_table=abi.ptr(table),
                             block_size=int(metadata.block_size), target_base=int(plan.owner) * self.history)
            rec.prefix_imported = True
            if plan.stop > plan.begin:
                spans.append(np.arange(plan.begin, plan.stop, dtype=np.int64))
                bases.append(np.full(plan.stop - plan.begin, int(plan.owner) * self.history, np.int64))
        if not spans:
            return
        tokens = torch.from_numpy(np.concatenate(spans)).to(self.device)
        sources = metadata.slot_mapping.to(torch.int64).index_select(0, tokens).contiguous()
        targets = (positions.to(torch.int64).index_select(0, tokens) +
                   torch.from_numpy(np.concatenate(bases)).to(self.device)).contiguous()
        self._launch(rows, mode=abi.INGEST_LIST, count=int(tokens.numel()), sources=abi.ptr(sources),
                     targets=abi.ptr(targets), target_base=0)

    def ingest_decode(self, cache, metadata, inputs, row_owners):
        """Graph-safe step: the packed rows of `inputs` (QueryInputs) each move one index-K
        row, live rows to (owner, query_end - 1), padding rows to distinct positions of owner
        0. Only batch * 4 rows move, whatever the history."""
        rows = self._paged_rows(cache)
        slots = metadata.slot_mapping
        if slots.dtype != self.torch.int64 or not slots.is_contiguous():
            raise ValueError("decode ingestion reads a contiguous int64 slot_mapping")
        if row_owners.dtype != self.torch.int32 or not row_owners.is_contiguous():
            raise ValueError("decode ingestion reads contiguous int32 row owners")
        self._launch(rows, mode=abi.INGEST_DECODE, count=inputs.query_ends.numel(),
                     query_ends=abi.ptr(inputs.query_ends), gather_indices=abi.ptr(inputs.gather_indices),
                     slot_mapping=abi.ptr(slots), slot_count=slots.numel(), row_owners=abi.ptr(row_owners),
                     queries_per_request=4, history=self.history)


# The reference exports the adapter subclass under the storage's name as well.
IndexCacheStorage = VllmIndexCacheStorage
