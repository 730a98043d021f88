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


class _StepLayout:
    """Host view of one scheduler step: its plans split by kind, the decode requests' query
    layout, and the step kind ("decode": no plan or decode plans only; "prefill": prefill
    plans only; "mixed")."""

    __slots__ = ("plans", "decodes", "prefills", "kind")

    def __init__(self, plans=()):
        self.plans = tuple(plans)
        self.decodes = tuple(p for p in self.plans if p.decode)
        self.prefills = tuple((row, p) for row, p in enumerate(self.plans) if not p.decode)
        if self.prefills:
            self.kind = "mixed" if self.decodes else "prefill"
        else:
            self.kind = "decode"

    def query_layout(self):
        """(query counts, first flat token, owner row) of every decode request, in order."""
        counts, begins, owners = [], [], []
        for p in self.decodes:
            counts.append(int(p.stop - p.begin))
            begins.append(int(p.begin))
            owners.append(int(p.owner))
        return counts, begins, owners

    def shared_decode_owners(self):
        """Owner rows named by more than one decode request that has tokens this step."""
        seen, shared = set(), set()
        for p in self.decodes:
            if p.stop > p.begin:
                (shared if p.owner in seen else seen).add(p.owner)
        return sorted(shared)


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
        self.torch, self.inputs, self.rotating, self.update, self.storage = torch, inputs, rotating, update, storage
        self.logical_ids, self.row_owners, self.prefix_workspace = logical_ids, row_owners, prefix_workspace
        self.unique_active_owners = unique_active_owners
        self.forward = forward_factory(rotating, update)
        self.history = int(logical_ids.shape[1])
        self.topk = rotating.topk.view(inputs.batch, QUERIES_PER_REQUEST, TOPK)
        # A row-owner tensor of its own is refreshed from the inputs' row by every prepare.
        self._owners_copied = row_owners.data_ptr() != inputs.row_owners.data_ptr()
        self._step = _StepLayout()
        self._selection = None  # hot-cache slots of the last decode selection, token order
        # Caller-set per step: positions of the step's tokens (the prefill Index ingest
        # reads them), and the ABC tail bounds ([batch, 2] int32 {begin, end}, e.g. columns
        # 2:4 of the serving policy's ABC descriptors) copied into the update's tail_bounds
        # before each decode forward (selector.py:42, :115-116 of the reference).
        self.positions = None
        self.tail_source = None

    # The step's plans as the reference's selector exposes them.
    plans = property(lambda self: self._step.plans or None)
    decodes = property(lambda self: self._step.decodes)
    prefills = property(lambda self: self._step.prefills)
    attention_indices = property(lambda self: self._selection)

    def prepare(self, plans, *, prepare_inputs=True):
        """Host layout of one scheduler step, no device read: the Index owners of new
        requests are reset and the decode requests' query rows laid out."""
        step = _StepLayout(plans)
        if self.unique_active_owners:
            shared = step.shared_decode_owners()
            if shared:
                raise ValueError(f"decode requests share an owner row: {shared}")
        self._step = step
        if self.storage is not None:
            self.storage.prepare(step.plans)
        if prepare_inputs:
            counts, begins, owners = step.query_layout()
            self.inputs.prepare(counts, query_starts=begins, query_owners=owners)
        if self._owners_copied:
            self.row_owners.copy_(self.inputs.row_owners)

    def __call__(self, query, weights, indexer, metadata, query_scale):
        """TopK-2048 logical positions of the step's tokens, int32 [tokens, 1, 2048]; the
        slots of the decode tokens' selections are kept for `slots`."""
        step = self._step
        self._ingest(step, indexer, metadata)
        if step.kind == "prefill":
            return indexer.select_topk_native(query, weights, metadata, query_scale)
        tokens = int(weights.shape[0])
        logical = self._decode(query, weights, query_scale, step, tokens)
        if step.kind == "decode":
            return logical
        return self._mixed(query, weights, query_scale, indexer, metadata, logical, tokens)

    def _ingest(self, step, indexer, metadata):
        """Index rows of the step's new tokens: the prefill list (restored prefixes first)
        when the step holds prefill requests, else the decode rows of the packed inputs."""
        if self.storage is None:
            return
        cache = indexer.k_cache.kv_cache
        if step.prefills:
            self.storage.ingest_prefill(cache, metadata, step.plans, self.positions)
        else:
            self.storage.ingest_decode(cache, metadata, self.inputs, self.row_owners)

    def _decode(self, query, weights, query_scale, step, tokens):
        """The resident LIFetch forward over the packed decode rows; its token-order outputs
        (logical positions returned, hot-cache slots kept for `slots`)."""
        self.inputs.pack(query, weights, query_scale)
        if self.tail_source is not None:
            if self.update.tail_bounds is None:
                raise ValueError("tail_source needs a ResidentIndexUpdate bound with tail_bounds")
            self.update.tail_bounds.copy_(self.tail_source)
        self.forward()
        # A decode-only batch that fits the packed capacity publishes one row per token; a
        # mixed or larger batch publishes the packed decode tokens first.
        packed = step.kind == "mixed" or tokens > self.inputs.capacity
        live = self.inputs.token_count if packed else tokens
        self._selection = self.update.slot_output.narrow(0, 0, live)
        return self.update.logical_output.narrow(0, 0, live)

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
        held = self._selection
        if held is None:
            raise RuntimeError("slots() needs a selection: call the selector for this step first")
        available = int(held.shape[0])
        if not 0 <= token_count <= available:
            raise ValueError(f"{token_count} tokens requested, the last selection holds {available}")
        return held.narrow(0, 0, token_count)
