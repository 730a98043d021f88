"""Fixed decode query buffers for LIFetch, filled from vLLM's packed token batch.

Mirrors the reference's `QueryInputs` (python/kvip/adapters/vllm/inputs.py:38-152):
the same constructor, `prepare` / `bind_positions` / `pack`, shapes, dtypes and
ValueError checks. `prepare` is host work (numpy on pinned staging, one H2D copy of the
five metadata rows); `bind_positions` and `pack` are one HIP launch each
(`kvip_hip_pack_queries`), graph-capturable, writing the persistent buffers in place.
"""
from __future__ import annotations

import ctypes

import numpy as np

from kvip_amd.runtime import abi

QUERIES_PER_REQUEST = 4
INDEX_WIDTH = 128


def committed_candidates(candidates, committed, resident):
    """Keep Index permutations inside the committed prefix (inputs.py:16-29): entries
    below min(committed, resident) first, then the missing committed rows in order,
    then the rest, truncated to the input length."""
    limit = min(committed, resident)
    if limit == resident:
        return candidates
    eligible = candidates[candidates < limit]
    missing = np.setdiff1d(np.arange(limit, dtype=np.int32), eligible, assume_unique=True)
    return np.concatenate((eligible, missing, candidates[candidates >= limit]))[: len(candidates)]


class QueryInputs:
    def __init__(self, torch, batch, device, *, pin_memory=True, history=0, index_heads=64):
        if index_heads not in (32, 64):
            raise ValueError("LIFetch supports 32 or 64 Indexer heads")
        self.index_heads = index_heads
        self.torch, self.batch, self.device = torch, batch, abi.device_of(torch, device)
        capacity = batch * QUERIES_PER_REQUEST
        # Rows: gather indices, query validity, unpack indices, output validity, row owners
        # (int32 pairs in the last int64 row), uploaded together.
        self.metadata = torch.zeros((5, capacity), dtype=torch.int64, device=self.device)
        self.host = [torch.zeros((5, capacity), dtype=torch.int64, pin_memory=pin_memory) for _ in range(2)]
        self.host_events = [None, None]
        self.turn = 0
        self.gather_indices, self.query_valid, self.unpack_indices, self.output_valid = self.metadata[:4].unbind(0)
        self.row_owners = self.metadata[4].view(torch.int32)[:batch]
        self.query = torch.zeros((capacity, index_heads, INDEX_WIDTH), dtype=torch.float8_e4m3fn, device=self.device)
        self.weights = torch.zeros((capacity, index_heads), dtype=torch.bfloat16, device=self.device)
        self.scale = torch.zeros((capacity, index_heads), dtype=torch.float32, device=self.device)
        self.query_ends = torch.zeros(capacity, dtype=torch.int32, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.token_count = 0
        self.block_offsets = torch.arange(history // 128, dtype=torch.int32, device=self.device)
        self.block_table = torch.zeros((batch, history // 128), dtype=torch.int32, device=self.device)
        self.block_bases = torch.zeros((batch, 1), dtype=torch.int32, device=self.device)

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (
            self.metadata, self.query, self.weights, self.scale, self.query_ends, self.block_offsets,
            self.block_table, self.block_bases))

    def prepare(self, query_counts, *, query_starts=None, query_owners=None):
        """Host packing of one scheduler batch (inputs.py:75-125), outside capture: row
        slot start = 4 * request, gather index = token of that query, unpack index = slot
        of each token, validities, owners; uploaded with one non-blocking copy."""
        counts = tuple(query_counts)
        if len(counts) > self.batch or any(type(n) is not int or not 0 <= n <= 4 for n in counts):
            raise ValueError("LIFetch rows require zero to four queries per request")
        starts = None if query_starts is None else tuple(query_starts)
        if starts is not None and (len(starts) != len(counts) or any(type(n) is not int or n < 0 for n in starts)):
            raise ValueError("Decode query starts must match request rows and be nonnegative")
        owners = None if query_owners is None else tuple(query_owners)
        if owners is not None and (
            len(owners) != len(counts) or any(type(n) is not int or not 0 <= n < (1 << 31) for n in owners)
        ):
            raise ValueError("Decode owners must match request rows and fit nonnegative int32")
        ring = self.turn % 2
        event = self.host_events[ring]
        if event is not None and not event.query():
            event.synchronize()
        values = self.host[ring].numpy()
        values.fill(0)
        if owners is not None:
            self.host[ring][4].view(self.torch.int32)[: len(owners)].numpy()[...] = owners
        begin = 0
        for row, count in enumerate(counts):
            slot = row * QUERIES_PER_REQUEST
            source = begin if starts is None else starts[row]
            values[0, slot:slot + count] = np.arange(source, source + count)
            values[1, slot:slot + count] = 1
            values[2, begin:begin + count] = np.arange(slot, slot + count)
            values[3, begin:begin + count] = 1
            begin += count
        self.token_count = begin
        self.metadata.copy_(self.host[ring], non_blocking=True)
        if self.block_offsets.numel():
            self.torch.mul(self.row_owners[:, None], self.block_offsets.numel(), out=self.block_bases)
            self.torch.add(self.block_bases, self.block_offsets, out=self.block_table)
        if self.device.type == "cuda":
            if self.host_events[ring] is None:
                self.host_events[ring] = self.torch.cuda.Event()
            self.host_events[ring].record(self.torch.cuda.current_stream(self.device))
        self.turn += 1

    def _launch(self, tokens, positions=None, query=None, weights=None, scale=None):
        if self.device.type != "cuda":
            raise ValueError("QueryInputs device work needs GPU tensors (kvip_amd has no CPU path)")
        torch = self.torch
        lib = abi.load_library()
        p = abi.ptr
        args = abi.QueryPackArgs(
            gather_indices=p(self.gather_indices), query_valid=p(self.query_valid), positions=p(positions),
            query_ends=p(self.query_ends), query_in=p(query), weights_in=p(weights), scale_in=p(scale),
            query_out=p(self.query) if query is not None else 0, weights_out=p(self.weights) if query is not None else 0,
            scale_out=p(self.scale) if query is not None else 0, status=p(self.status), tokens=tokens,
            rows=self.batch * QUERIES_PER_REQUEST, heads=self.index_heads,
        )
        abi.check(lib.kvip_hip_pack_queries(ctypes.byref(args), abi.stream_handle(torch, self.device)),
                  "pack_queries")

    def bind_positions(self, positions):
        """query_ends[row] = (positions[gather] + 1) * valid (inputs.py:127-133), after
        the runner's MTP position correction; returns the [batch, 4] view."""
        if positions.dim() != 1 or positions.dtype != self.torch.int64 or positions.device != self.device:
            raise ValueError("LIFetch positions must be int64 [tokens] on the inputs' device")
        self._launch(positions.shape[0], positions=positions.contiguous())
        return self.query_ends.view(self.batch, QUERIES_PER_REQUEST)

    def pack(self, query, weights, scale):
        """Graph-safe byte gather of the token batch's index Q, weights and scales into
        the fixed [batch*4, ...] buffers (inputs.py:135-152)."""
        if weights.ndim != 2 or weights.shape[1] != self.index_heads:
            raise ValueError("LIFetch weights require [tokens,index_heads]")
        tokens = weights.shape[0]
        if tuple(query.shape) == (tokens * self.index_heads, INDEX_WIDTH):
            query = query.view(tokens, self.index_heads, INDEX_WIDTH)
        if tuple(query.shape) != (tokens, self.index_heads, INDEX_WIDTH) or query.dtype != self.query.dtype:
            raise ValueError("LIFetch requires FP8 e4m3 Index queries with the configured head count and width 128")
        if scale is None or scale.dtype != self.scale.dtype or weights.dtype != self.weights.dtype:
            raise ValueError("LIFetch requires float32 query scales and BF16 weights")
        if tuple(scale.shape) in ((tokens * self.index_heads,), (tokens * self.index_heads, 1)):
            scale = scale.view(tokens, self.index_heads)
        if tuple(scale.shape) != (tokens, self.index_heads):
            raise ValueError("LIFetch requires one scale per token/head")
        for t in (query, weights, scale):
            if not t.is_contiguous() or t.device != self.device or t.data_ptr() % 16:
                raise ValueError("LIFetch query inputs must be contiguous, 16-byte aligned and on the inputs' device")
        self._launch(tokens, query=query, weights=weights, scale=scale)
        return self.query, self.weights, self.scale
