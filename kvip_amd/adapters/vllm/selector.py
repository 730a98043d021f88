"""vLLM indexer selector over service-owned LIFetch inputs and Index updates.

Interface of the reference's VllmIndexSelector (python/kvip/adapters/vllm/selector.py:
46-161): built over a QueryInputs, a LIFetch binding reading them, an Index update and
the storage's logical ids; `prepare(plans)` once per scheduler step on the host (no
device read), `__call__(query, weights, indexer, metadata, query_scale)` returning the
step's TopK-2048 logical positions per token, int32 [tokens, 1, 2048], and
`slots(token_count)` returning the hot-cache slots the sparse attention reads.

Step kinds, as in the reference: decode-only steps run the Index ingest, the query
packing and the resident LIFetch forward, whose update publishes logical and slot
outputs in token order; prefill-only steps go to the indexer's native selection;
mixed steps do both. Design of the mixed step on MI355X: all prefill requests of the
step are packed as the sequences of one TND prefill launch (their token rows gathered,
cumulative query lengths, key lengths and block-table rows stacked), instead of one
native call per request, and the two halves land in token order with one scatter each.

`RequestPlan` names the fields of a scheduled request that the selector and the Index
storage read. `PagedIndexer` is the indexer side on MI355X: the paged index-K cache the
storage imports from (`k_cache.kv_cache`) and `select_topk_native`, the prefill lightning
indexer with TopK-2048 over that cache (`kvip_amd.PrefillIndexer`), in the place of the
native indexer call the reference's vLLM build makes.
"""
from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace
from typing import Any

import numpy as np

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

    @property
    def max_sequences(self):
        return self.prefill.max_sequences

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
        """inputs: QueryInputs; rotating: a LIFetchBinding reading them
        (`bind_query_inputs`); update: a ResidentIndexUpdate publishing token-order
        outputs of those inputs; logical_ids: the storage's int64 [owners, history];
        row_owners: int32 [batch], the inputs' owner row or a copy refreshed by prepare;
        storage: the VllmIndexCacheStorage ingested into (None: the caller ingests)."""
        problems = []
        if logical_ids.ndim != 2 or logical_ids.dtype != torch.int64 or not logical_ids.is_contiguous():
            problems.append("logical ids must be contiguous int64 [owners, history]")
        if tuple(row_owners.shape) != (inputs.batch,) or row_owners.dtype != torch.int32:
            problems.append(f"row owners must be int32 [{inputs.batch}]")
        if rotating.batch != inputs.batch or rotating.rows_per_request != QUERIES_PER_REQUEST:
            problems.append(f"the binding must hold {inputs.batch} requests x {QUERIES_PER_REQUEST} query rows")
        bound = {"query": (rotating.query, inputs.query), "weights": (rotating.weights, inputs.weights),
                 "query scale": (rotating.query_scale, inputs.scale)}
        for name, (have, want) in bound.items():
            if have is None or have.data_ptr() != want.data_ptr():
                problems.append(f"the binding's {name} is not the packed QueryInputs buffer")
        if not isinstance(update, ResidentIndexUpdate) or update.query_inputs is not inputs:
            problems.append("the Index update must publish token-order outputs of these QueryInputs")
        if problems:
            raise ValueError("VllmIndexSelector: " + "; ".join(problems))
        self.torch, self.inputs, self.rotating, self.update = torch, inputs, rotating, update
        self.forward = forward_factory(rotating, update)
        self.unique_active_owners = unique_active_owners
        self.logical_ids, self.row_owners = logical_ids, row_owners
        self.prefix_workspace = prefix_workspace
        self.storage, self.positions = storage, None
        self.history = int(logical_ids.shape[1])
        self.topk = rotating.topk.view(inputs.batch, QUERIES_PER_REQUEST, TOPK)
        self.attention_indices = None
        # ABC tail bounds of the step ([batch, 2] int32 {begin, end}, e.g. columns 2:4 of the
        # serving policy's ABC descriptors), copied into the update's tail_bounds before each
        # decode forward (selector.py:42, :115-116 of the reference).
        self.tail_source = None
        self.plans = None
        self.decodes = ()
        self.prefills = ()

    def prepare(self, plans, *, prepare_inputs=True):
        """Host layout of one scheduler step, no device read: the Index owners of new
        requests are reset and the decode requests' query rows laid out."""
        self.plans = tuple(plans)
        self.decodes = tuple(p for p in self.plans if p.decode)
        self.prefills = tuple((row, p) for row, p in enumerate(self.plans) if not p.decode)
        if self.unique_active_owners:
            live = [p.owner for p in self.decodes if p.stop > p.begin]
            if len(set(live)) != len(live):
                raise ValueError(f"decode requests share an owner row: {sorted(live)}")
        if self.storage is not None:
            self.storage.prepare(self.plans)
        if prepare_inputs:
            self.inputs.prepare([int(p.stop - p.begin) for p in self.decodes],
                                query_starts=[int(p.begin) for p in self.decodes],
                                query_owners=[int(p.owner) for p in self.decodes])
        if self.row_owners.data_ptr() != self.inputs.row_owners.data_ptr():
            self.row_owners.copy_(self.inputs.row_owners)

    def __call__(self, query, weights, indexer, metadata, query_scale):
        """TopK-2048 logical positions of the step's tokens, int32 [tokens, 1, 2048]; the
        slots of the decode tokens' selections are kept for `slots`."""
        mixed = bool(self.decodes) and bool(self.prefills)
        if self.storage is not None:
            cache = indexer.k_cache.kv_cache
            if self.prefills:
                self.storage.ingest_prefill(cache, metadata, self.plans, self.positions)
            else:
                self.storage.ingest_decode(cache, metadata, self.inputs, self.row_owners)
        if self.plans and not self.decodes:
            return indexer.select_topk_native(query, weights, metadata, query_scale)
        self.inputs.pack(query, weights, query_scale)
        if self.tail_source is not None:
            if self.update.tail_bounds is None:
                raise ValueError("tail_source needs a ResidentIndexUpdate bound with tail_bounds")
            self.update.tail_bounds.copy_(self.tail_source)
        self.forward()
        tokens = int(weights.shape[0])
        live = self.inputs.token_count if mixed or tokens > self.inputs.capacity else tokens
        logical = self.update.logical_output[:live]
        self.attention_indices = self.update.slot_output[:live]
        if not mixed:
            return logical
        return self._mixed(query, weights, query_scale, indexer, metadata, logical, tokens)

    def _mixed(self, query, weights, query_scale, indexer, metadata, logical, tokens):
        """Token-order result of a mixed step: the decode tokens' published rows and one
        batched native selection per group of at most `indexer.max_sequences` prefill
        requests."""
        torch, dev = self.torch, weights.device
        heads = self.inputs.index_heads
        result = torch.full((tokens, 1, TOPK), -1, dtype=torch.int32, device=dev)
        dec = np.concatenate([np.arange(p.begin, p.stop) for p in self.decodes]).astype(np.int64)
        if dec.size:
            result.index_copy_(0, torch.from_numpy(dec).to(dev), logical[:dec.size].reshape(dec.size, 1, TOPK))
        q_rows = query.reshape(tokens, heads, INDEX_DIM)
        s_rows = query_scale.reshape(tokens, heads)
        group = getattr(indexer, "max_sequences", len(self.prefills))
        for g0 in range(0, len(self.prefills), group):
            part = self.prefills[g0:g0 + group]
            counts = np.array([p.stop - p.begin for _, p in part], np.int64)
            rows = np.concatenate([np.arange(p.begin, p.stop) for _, p in part]).astype(np.int64)
            if rows.size == 0:
                continue
            rows_d = torch.from_numpy(rows).to(dev)
            packed = SimpleNamespace(
                block_size=getattr(metadata, "block_size", BLOCK_TOKENS),
                block_table=metadata.block_table.index_select(
                    0, torch.tensor([r for r, _ in part], dtype=torch.int64, device=dev)),
                cum_query_lens=torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(dev),
                seq_lens=torch.cat([p.key_end.reshape(-1).to(torch.int32) for _, p in part]))
            packed.actual_seq_lengths_query = packed.cum_query_lens
            packed.actual_seq_lengths_key = packed.seq_lens
            selected = indexer.select_topk_native(q_rows.index_select(0, rows_d), weights.index_select(0, rows_d),
                                                  packed, s_rows.index_select(0, rows_d))
            result.index_copy_(0, rows_d, selected.reshape(rows.size, 1, TOPK))
        return result

    def slots(self, token_count):
        """Hot-cache slots of the last selection's first `token_count` decode tokens (the
        indices the sparse attention reads)."""
        if self.attention_indices is None:
            raise RuntimeError("slots() needs a selection: call the selector for this step first")
        if token_count > self.attention_indices.shape[0]:
            raise ValueError(f"{token_count} tokens requested, the last selection holds "
                             f"{self.attention_indices.shape[0]}")
        return self.attention_indices[:token_count]
