"""Fixed decode query buffers of the LIFetch path, filled from vLLM's flat token batch.

Interface of the reference's QueryInputs (python/kvip/adapters/vllm/inputs.py:38-152):
up to four query rows per request in packed rows [batch * 4]; the per-row fields
`gather_indices`, `query_valid`, `unpack_indices`, `output_valid` (int64) and
`row_owners` (int32), the packed `query` fp8 [batch * 4, heads, 128], `weights` bf16 and
`scale` fp32 [batch * 4, heads], `query_ends` int32 [batch * 4] (position + 1, 0 =
padding) and the owners' Index block table; `prepare(query_counts, query_starts=,
query_owners=)` on the host before the step, `bind_positions(positions)` and
`pack(query, weights, scale)` on the device inside it.

Design. `prepare` lays a step out with vectorised numpy into one block of a ring of
pinned staging blocks and queues two copies: the five metadata rows (the owners ride in
the last int64 row as int32 pairs) and the owners' block table (row b = owner * blocks +
0, 1, ...). A staging block is rewritten only after the event recorded behind its copies
has completed, so the host never waits on the step it just queued. `bind_positions` and
`pack` are one `kvip_hip_pack_queries` launch each, graph-capturable, writing the
persistent buffers in place.
"""
from __future__ import annotations

import ctypes

import numpy as np

from kvip_amd.runtime import abi

QUERIES_PER_REQUEST = 4
INDEX_WIDTH = 128
BLOCK_TOKENS = 128
STAGING_DEPTH = 2


def committed_candidates(candidates, committed, resident):
    """LRU candidates confined to the committed Index prefix (the reference's rule,
    inputs.py:16-29). Below the resident size only positions < min(committed, resident)
    may become destinations: candidates inside that prefix keep their order, the prefix
    positions no candidate names follow in ascending order, then the rest; the result
    keeps the input length. At full residency the input itself is returned."""
    limit = min(int(committed), int(resident))
    if limit >= resident:
        return candidates
    cand = np.asarray(candidates)
    inside = cand < limit
    named = np.zeros(limit, dtype=bool)
    named[cand[inside & (cand >= 0)]] = True
    unnamed = np.flatnonzero(~named).astype(cand.dtype)
    return np.concatenate((cand[inside], unnamed, cand[~inside]))[:cand.size]


def _ints(values, what, low, high):
    out = tuple(values)
    for v in out:
        if type(v) is not int or not low <= v < high:
            raise ValueError(f"{what}: expected Python ints in [{low}, {high}), got {v!r}")
    return out


class QueryInputs:
    def __init__(self, torch, batch, device, *, pin_memory=True, history=0, index_heads=64):
        if index_heads not in (32, 64):
            raise ValueError(f"index heads must be 32 or 64 (got {index_heads})")
        if batch < 1:
            raise ValueError(f"batch must be positive (got {batch})")
        self.torch, self.batch, self.index_heads = torch, int(batch), int(index_heads)
        self.device = abi.device_of(torch, device)
        self.capacity = rows = self.batch * QUERIES_PER_REQUEST
        self.blocks = int(history) // BLOCK_TOKENS
        dev = self.device
        self.metadata = torch.zeros((5, rows), dtype=torch.int64, device=dev)
        self.gather_indices, self.query_valid, self.unpack_indices, self.output_valid = self.metadata[:4].unbind(0)
        self.row_owners = self.metadata[4].view(torch.int32)[:self.batch]
        self.block_table = torch.zeros((self.batch, self.blocks), dtype=torch.int32, device=dev)
        self.query = torch.zeros((rows, index_heads, INDEX_WIDTH), dtype=torch.float8_e4m3fn, device=dev)
        self.weights = torch.zeros((rows, index_heads), dtype=torch.bfloat16, device=dev)
        self.scale = torch.zeros((rows, index_heads), dtype=torch.float32, device=dev)
        self.query_ends = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self._staging = [(torch.zeros((5, rows), dtype=torch.int64, pin_memory=pin_memory),
                          torch.zeros((self.batch, self.blocks), dtype=torch.int32, pin_memory=pin_memory))
                         for _ in range(STAGING_DEPTH)]
        self._events = [None] * STAGING_DEPTH
        self._steps = 0
        self._ramp = np.arange(self.blocks, dtype=np.int32)
        self.token_count = 0

    @property
    def nbytes(self):
        """Device bytes of the persistent buffers."""
        return sum(t.numel() * t.element_size() for t in (
            self.metadata, self.block_table, self.query, self.weights, self.scale, self.query_ends, self.status))

    def prepare(self, query_counts, *, query_starts=None, query_owners=None):
        """Host layout of one scheduler step, outside capture, no device read. Request r
        owns packed rows 4r .. 4r + count_r - 1; its tokens come at token offset
        query_starts[r] (default: consecutive in request order) of the flat batch."""
        counts = _ints(query_counts, "query counts", 0, QUERIES_PER_REQUEST + 1)
        if len(counts) > self.batch:
            raise ValueError(f"{len(counts)} requests exceed the bound batch of {self.batch}")
        starts = None if query_starts is None else _ints(query_starts, "query starts", 0, 1 << 62)
        owners = None if query_owners is None else _ints(query_owners, "query owners", 0, 1 << 31)
        for name, seq in (("query starts", starts), ("query owners", owners)):
            if seq is not None and len(seq) != len(counts):
                raise ValueError(f"{name}: {len(seq)} entries for {len(counts)} requests")
        k = self._steps % STAGING_DEPTH
        if self._events[k] is not None:
            self._events[k].synchronize()
        meta_t, table_t = self._staging[k]
        meta = meta_t.numpy()
        meta.fill(0)
        n = np.asarray(counts, dtype=np.int64)
        total = int(n.sum())
        request = np.repeat(np.arange(len(n)), n)
        within = np.arange(total) - np.repeat(np.cumsum(n) - n, n)
        rows = request * QUERIES_PER_REQUEST + within
        tokens = np.arange(total) if starts is None else np.repeat(np.asarray(starts, np.int64), n) + within
        meta[0, rows] = tokens
        meta[1, rows] = 1
        meta[2, :total] = rows
        meta[3, :total] = 1
        own = np.zeros(self.batch, dtype=np.int32)
        if owners is not None:
            own[:len(owners)] = owners
        meta_t[4].view(self.torch.int32).numpy()[:self.batch] = own
        table_t.numpy()[...] = own[:, None] * self.blocks + self._ramp[None, :]
        self.metadata.copy_(meta_t, non_blocking=True)
        self.block_table.copy_(table_t, non_blocking=True)
        if self.device.type == "cuda":
            if self._events[k] is None:
                self._events[k] = self.torch.cuda.Event()
            self._events[k].record(self.torch.cuda.current_stream(self.device))
        self.token_count = total
        self._steps += 1

    def _launch(self, tokens, positions=None, query=None, weights=None, scale=None):
        if self.device.type != "cuda":
            raise ValueError("query packing runs on the GPU only (kvip_amd has no CPU path)")
        p = abi.ptr
        gather = query is not None
        args = abi.QueryPackArgs(
            gather_indices=p(self.gather_indices), query_valid=p(self.query_valid), positions=p(positions),
            query_ends=p(self.query_ends), query_in=p(query), weights_in=p(weights), scale_in=p(scale),
            query_out=p(self.query) if gather else 0, weights_out=p(self.weights) if gather else 0,
            scale_out=p(self.scale) if gather else 0, status=p(self.status), tokens=tokens, rows=self.capacity,
            heads=self.index_heads)
        abi.check(abi.load_library().kvip_hip_pack_queries(ctypes.byref(args),
                                                           abi.stream_handle(self.torch, self.device)),
                  "kvip_hip_pack_queries")

    def bind_positions(self, positions):
        """query_ends[row] = (positions[gather_indices[row]] + 1) * query_valid[row], once per
        step after the runner's MTP position correction; returns the [batch, 4] view."""
        torch = self.torch
        if positions.dim() != 1 or positions.dtype != torch.int64 or positions.device != self.device:
            raise ValueError("positions must be an int64 vector of the step's tokens on the inputs' device")
        self._launch(int(positions.shape[0]), positions=positions.contiguous())
        return self.query_ends.view(self.batch, QUERIES_PER_REQUEST)

    def pack(self, query, weights, scale):
        """Gather the step's index queries (fp8 [tokens, heads, 128], or flattened to
        [tokens * heads, 128]), bf16 weights [tokens, heads] and fp32 scales ([tokens,
        heads], [tokens * heads] or [tokens * heads, 1]) into the packed rows."""
        torch, heads = self.torch, self.index_heads
        if weights.ndim != 2 or weights.shape[1] != heads or weights.dtype != torch.bfloat16:
            raise ValueError(f"weights must be bf16 [tokens, {heads}] (got {weights.dtype}, {tuple(weights.shape)})")
        tokens = int(weights.shape[0])
        if query.dtype != torch.float8_e4m3fn or query.numel() != tokens * heads * INDEX_WIDTH:
            raise ValueError(f"queries must be fp8 e4m3 holding [{tokens}, {heads}, {INDEX_WIDTH}] "
                             f"(got {query.dtype}, {tuple(query.shape)})")
        if query.shape[-1] != INDEX_WIDTH:
            raise ValueError(f"queries must end in the index width {INDEX_WIDTH} (got {tuple(query.shape)})")
        if scale is None or scale.dtype != torch.float32 or scale.numel() != tokens * heads:
            raise ValueError(f"query scales must be float32 holding one value per token and head")
        if tuple(scale.shape) not in ((tokens, heads), (tokens * heads,), (tokens * heads, 1)):
            raise ValueError(f"query scales of shape {tuple(scale.shape)} do not name [tokens, heads]")
        for t in (query, weights, scale):
            if not t.is_contiguous() or t.device != self.device or t.data_ptr() % 16:
                raise ValueError("query inputs must be contiguous, 16-byte aligned and on the inputs' device")
        self._launch(tokens, query=query, weights=weights, scale=scale)
        return self.query, self.weights, self.scale
