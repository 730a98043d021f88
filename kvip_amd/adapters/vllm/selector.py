"""vLLM indexer selector over service-owned LIFetch inputs and Index updates.

Mirrors the reference's VllmIndexSelector (python/kvip/adapters/vllm/selector.py:46-161):
the same constructor checks, `prepare(plans)` (host request layout, once per step, no
device readback), `__call__(query, weights, indexer, metadata, query_scale)` and
`slots(token_count)`. A step of decode requests runs Index ingest (one
`kvip_hip_ingest_index` launch), the packing of the token batch's index queries into the
fixed [batch * 4] rows (`kvip_hip_pack_queries`) and the resident LIFetch forward, whose
Index update publishes the logical and slot TopK in token order; nothing is gathered,
cast or masked afterwards. Prefill-only steps go to the indexer's native selection, and
mixed steps run the forward for the decode requests and the native selection for each
prefill request, assembled in token order.

`RequestPlan` names the fields of a scheduled request that the selector and the Index
storage read. `PagedIndexer` is the indexer side on MI355X: the paged index-K cache the
storage imports from (`k_cache.kv_cache`) and `select_topk_native`, the prefill lightning
indexer with TopK-2048 over that cache (`kvip_amd.PrefillIndexer`), in the place of the
native indexer call the reference's vLLM build makes.
"""
from __future__ import annotations

from copy import copy
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Any

from kvip_amd.operators.lifetch.forward import LIFetchForward
from kvip_amd.operators.lifetch.resident import ResidentIndexUpdate
from kvip_amd.operators.prefill import PrefillIndexer

TOPK = 2048
QUERIES_PER_REQUEST = 4
BLOCK_TOKENS = 128
INDEX_DIM = 128


@dataclass(frozen=True)
class RequestPlan:
    """One request of a scheduler step, as the selector (selector.py:87-154) and the Index
    storage (cache/index_storage.py:36-46, adapters/vllm/index_import.py:17-36) read it.

    owner      stable Index owner row of the request;
    request    request id (a new id on an owner resets that owner's Index metadata);
    begin/stop the request's tokens in the step's flat token batch;
    start      positions already in the paged cache before the step (restored prefix);
    decode     True for a decode request (one to four query tokens);
    query_end / key_end  prefill metadata of the request: int32 device tensors [1] holding
               the query count (cumulative query length of a one-sequence batch) and the
               context length after the step."""
    owner: int
    request: Any
    begin: int
    stop: int
    start: int = 0
    decode: bool = True
    query_end: Any = None
    key_end: Any = None


class PagedIndexer:
    """Paged index-K cache and native prefill selection of one attention layer.

    keys [blocks, 128, 128] float8_e4m3fn (or uint8 bytes), scales [blocks, 128] float32:
    vLLM's indexer cache with 128-token blocks. `select_topk_native(query, weights,
    metadata, query_scale)` scores packed query rows of `S` prefill sequences against
    their pages (metadata.block_table [S, blocks] int32, metadata.cum_query_lens [S]
    cumulative query counts and metadata.seq_lens [S] context lengths, int32 on the
    device) under the right-down causal mask and returns the TopK-2048 positions of each
    row within its sequence, int32 [rows, 1, 2048] (-1 padded). The returned tensor is
    this object's buffer, valid until the next call; the call allocates nothing."""

    def __init__(self, torch, *, keys, scales, max_rows, max_context, device, heads=64, max_sequences=1):
        if keys.dim() != 3 or tuple(keys.shape[1:]) != (BLOCK_TOKENS, INDEX_DIM) or keys.element_size() != 1:
            raise ValueError("paged index-K cache must be 1-byte [blocks, 128, 128]")
        if scales.dtype != torch.float32 or tuple(scales.shape) != tuple(keys.shape[:2]):
            raise ValueError("paged index-K scales must be float32 [blocks, 128]")
        self.torch = torch
        self.keys = keys if keys.dtype == torch.float8_e4m3fn else keys.view(torch.float8_e4m3fn)
        self.scales = scales
        self.k_cache = SimpleNamespace(kv_cache=(keys, scales))
        self.prefill = PrefillIndexer(torch, max_rows=max_rows, max_context=max_context, max_sequences=max_sequences,
                                      device=device, heads=heads, weight_dtype=torch.bfloat16)
        self.cu_seqlens = torch.zeros(max_sequences + 1, dtype=torch.int32, device=self.prefill.device)

    def select_topk_native(self, query, weights, metadata, query_scale):
        rows, heads = int(weights.shape[0]), self.prefill.heads
        ends = metadata.cum_query_lens.reshape(-1)
        sequences = int(ends.shape[0])
        if not 1 <= sequences <= self.prefill.max_sequences:
            raise ValueError("prefill metadata names more sequences than the indexer was built for")
        query = query.reshape(rows, heads, INDEX_DIM)
        if query.dtype == self.torch.uint8:
            query = query.view(self.torch.float8_e4m3fn)
        scale = None if query_scale is None else query_scale.reshape(rows, heads).contiguous()
        self.cu_seqlens[1:sequences + 1].copy_(ends)
        selected = self.prefill(query.contiguous(), weights.contiguous(), scale, self.keys, self.scales,
                                self.cu_seqlens[:sequences + 1], metadata.seq_lens.reshape(-1),
                                metadata.block_table)
        return selected.view(rows, 1, TOPK)


class VllmIndexSelector:
    def __init__(self, torch, *, inputs, rotating, update, logical_ids, row_owners, prefix_workspace=None,
                 storage=None, forward_factory=LIFetchForward, unique_active_owners=False):
        """inputs: QueryInputs; rotating: a LIFetchBinding that reads them
        (`bind_query_inputs`); update: a ResidentIndexUpdate publishing token-order
        outputs of those inputs; logical_ids: the storage's int64 [owners, history];
        row_owners: int32 [batch], the inputs' owner row or a copy refreshed by prepare;
        storage: the VllmIndexCacheStorage ingested into (None: the caller ingests)."""
        self.torch = torch
        self.inputs, self.rotating, self.update = inputs, rotating, update
        if logical_ids.ndim != 2 or not logical_ids.is_contiguous() or logical_ids.dtype != torch.int64:
            raise ValueError("LIFetch logical IDs require contiguous int64 owner/history rows")
        if tuple(row_owners.shape) != (inputs.batch,) or row_owners.dtype != torch.int32:
            raise ValueError("LIFetch row owners must match the bound batch")
        if rotating.batch != inputs.batch or rotating.rows_per_request != QUERIES_PER_REQUEST:
            raise ValueError("LIFetch locations and TopK must share the bound shape")
        for actual, expected in ((rotating.query, inputs.query), (rotating.weights, inputs.weights),
                                 (rotating.query_scale, inputs.scale)):
            if actual is None or actual.data_ptr() != expected.data_ptr():
                raise ValueError("LIFetch kernel must bind the persistent packed query buffers")
        if not isinstance(update, ResidentIndexUpdate) or update.query_inputs is not inputs:
            raise ValueError("LIFetch update must publish token-order outputs of the bound query inputs")
        self.forward = forward_factory(rotating, update)
        self.unique_active_owners = unique_active_owners
        self.logical_ids, self.row_owners = logical_ids, row_owners
        self.prefix_workspace = prefix_workspace
        self.storage, self.positions = storage, None
        self.topk = rotating.topk.view(inputs.batch, QUERIES_PER_REQUEST, TOPK)
        self.history = logical_ids.shape[1]
        self.attention_indices = None
        self.plans = None
        self.decodes = ()

    def prepare(self, plans, *, prepare_inputs=True):
        """Host request layout, once per step; no device readback (selector.py:87-104)."""
        self.plans = tuple(plans)
        self.decodes = tuple(p for p in self.plans if p.decode)
        if self.unique_active_owners:
            owners = [p.owner for p in self.decodes if p.stop > p.begin]
            if len(owners) != len(set(owners)):
                raise ValueError("active decode rows must have distinct stable owners")
        if self.storage is not None:
            self.storage.prepare(self.plans)
        if prepare_inputs:
            self.inputs.prepare([int(p.stop - p.begin) for p in self.decodes],
                                query_starts=[int(p.begin) for p in self.decodes],
                                query_owners=[int(p.owner) for p in self.decodes])
        if self.row_owners.data_ptr() != self.inputs.row_owners.data_ptr():
            self.row_owners.copy_(self.inputs.row_owners)

    def __call__(self, query, weights, indexer, metadata, query_scale):
        """TopK-2048 logical positions of the step's tokens, int32 [tokens, 1, 2048]
        (selector.py:106-154); the slot of every selected position is kept for `slots`."""
        mixed = self.plans is not None and len(self.decodes) != len(self.plans)
        if self.storage is not None:
            if mixed:
                self.storage.ingest_prefill(indexer.k_cache.kv_cache, metadata, self.plans, self.positions)
            else:
                self.storage.ingest_decode(indexer.k_cache.kv_cache, metadata, self.inputs, self.row_owners)
        if self.plans and not self.decodes:
            return indexer.select_topk_native(query, weights, metadata, query_scale)
        self.inputs.pack(query, weights, query_scale)
        self.forward()

        tokens = int(weights.shape[0])
        token_count = self.inputs.token_count if mixed or tokens > self.inputs.batch * QUERIES_PER_REQUEST else tokens
        logical = self.update.logical_output[:token_count]
        self.attention_indices = self.update.slot_output[:token_count]
        if not mixed:
            return logical

        # Prefill requests keep the paged Index cache and the native selection; decode rows
        # are not recomputed.
        torch = self.torch
        result = torch.full((tokens, 1, TOPK), -1, dtype=torch.int32, device=weights.device)
        heads = self.inputs.index_heads
        query_rows = query.view(tokens, heads, INDEX_DIM)
        scale_rows = query_scale.view(tokens, heads)
        offset = 0
        for row, plan in enumerate(self.plans):
            count = plan.stop - plan.begin
            if plan.decode:
                result[plan.begin:plan.stop].copy_(logical[offset:offset + count])
                offset += count
                continue
            prefill = copy(metadata)
            prefill.topk_selector = None
            prefill.num_actual_tokens = count
            prefill.block_table = metadata.block_table[row:row + 1]
            prefill.actual_seq_lengths_query = prefill.cum_query_lens = plan.query_end
            prefill.actual_seq_lengths_key = prefill.seq_lens = plan.key_end
            selected = indexer.select_topk_native(query_rows[plan.begin:plan.stop], weights[plan.begin:plan.stop],
                                                  prefill, scale_rows[plan.begin:plan.stop])
            result[plan.begin:plan.stop].copy_(selected.view(count, 1, TOPK))
        return result

    def slots(self, token_count):
        """Hot-cache slots of the last selection's first `token_count` tokens (the SFA
        consumer's indices, selector.py:156-161)."""
        if self.attention_indices is None:
            raise RuntimeError("LIFetch selection must execute before SFA")
        if token_count > self.attention_indices.shape[0]:
            raise ValueError("SFA query count exceeds the fused selection")
        return self.attention_indices[:token_count]
