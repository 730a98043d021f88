"""Buffers of one LIFetch pipeline, allocated once before capture.

`LIFetchBinding` is the MI355X-native `rotating` argument of ``kvip_amd.LIFetch``: it
owns the indexer inputs (query, weights, scales, request lengths, block table), the
score-key workspace and the TopK output, and is bound to a paged index-K cache.
`ContiguousFetch` is the `update` argument for a contiguous Fetch destination: it is
bound to a paged KV cache and owns the gathered [rows, 2048, row_bytes] buffer.

The reference's counterparts are LIFetchBinding (python/kvip/operators/lifetch/
binding.py:12-221) and LIFetchWorkspace (workspace.py:34-124), whose buffers feed the
14 LI argument pointers (workspace.py:105-124); here the same roles are plain device
tensors whose addresses go into the C ABI structs of include/kvip_hip.h.
"""
from __future__ import annotations

from kvip_amd.runtime import abi

TOPK = 2048
BLOCK_TOKENS = 128
INDEX_DIM = 128
TOKEN_BYTES = 656
TOPK_SEGMENT_KEYS = 2048
TOPK_SEGMENT_WORDS = 260
MAX_CONTEXT = 1 << 24


def _qk_dtype(torch, name):
    table = {"fp8": (torch.float8_e4m3fn, abi.DTYPE_FP8_E4M3), "bf16": (torch.bfloat16, abi.DTYPE_BF16)}
    if name not in table:
        raise ValueError(f"index Q/K dtype must be 'fp8' or 'bf16', not {name!r}")
    return table[name]


class LIFetchBinding:
    """Indexer inputs, workspace and TopK output for `batch` requests.

    rows = batch * rows_per_request query rows (1 for decode, up to 4 with MTP);
    max_context bounds every request's context (rounded up to 128-token blocks).
    The caller fills `query`, `weights`, `query_scale`, `seq_lens`, `block_table`
    (and `query_ends` when enabled) in place, then calls the LIFetch forward.
    """

    def __init__(self, torch, *, batch, max_context, device, heads=64, rows_per_request=1, qk_dtype="fp8",
                 weight_dtype=None, query_scale=True, query_ends=False):
        if not 1 <= batch <= 65535:
            raise ValueError(f"LIFetch batch must be in 1..65535, got {batch}")
        if heads not in (32, 64):
            raise ValueError("LIFetch supports 32 or 64 Indexer heads")
        if rows_per_request not in (1, 2, 4):
            raise ValueError("LIFetch supports 1, 2 or 4 query rows per request")
        if not 1 <= max_context <= MAX_CONTEXT:
            raise ValueError(f"max_context must be in 1..{MAX_CONTEXT}")
        weight_dtype = torch.float32 if weight_dtype is None else weight_dtype
        if weight_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("LIFetch weights must be float32 or bfloat16")
        self.torch, self.device = torch, abi.device_of(torch, device)
        self.batch, self.heads, self.rows_per_request = batch, heads, rows_per_request
        self.rows = batch * rows_per_request
        self.max_blocks = (max_context + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        self.key_stride = self.max_blocks * BLOCK_TOKENS
        self.qk_torch_dtype, self.qk_code = _qk_dtype(torch, qk_dtype)
        self.qk_name = qk_dtype
        self.weight_code = abi.DTYPE_FP32 if weight_dtype == torch.float32 else abi.DTYPE_BF16
        dev = self.device
        self.query = torch.zeros((self.rows, heads, INDEX_DIM), dtype=self.qk_torch_dtype, device=dev)
        self.weights = torch.zeros((self.rows, heads), dtype=weight_dtype, device=dev)
        self.query_scale = torch.ones((self.rows, heads), dtype=torch.float32, device=dev) if query_scale else None
        self.seq_lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.query_ends = torch.zeros(self.rows, dtype=torch.int32, device=dev) if query_ends else None
        self.block_table = torch.zeros((batch, self.max_blocks), dtype=torch.int32, device=dev)
        # int16 storage holding uint16 sortable keys (reinterpret with .view on the host).
        self.score_keys = torch.zeros((self.rows, self.key_stride), dtype=torch.int16, device=dev)
        self.histogram = torch.zeros((self.rows, 256), dtype=torch.int32, device=dev)
        # Per-segment records and per-row arrival counters of the multi-workgroup TopK
        # (zero once here; every launch leaves the counters at zero).
        segments = (self.key_stride + TOPK_SEGMENT_KEYS - 1) // TOPK_SEGMENT_KEYS
        self.topk_segments = torch.zeros((self.rows, segments, TOPK_SEGMENT_WORDS), dtype=torch.int32, device=dev)
        self.topk = torch.full((self.rows, TOPK), -1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.keys = None
        self.key_scale = None
        self.query_inputs = None

    def bind_index_cache(self, keys, key_scale=None):
        """Bind the paged index-K cache: keys [num_blocks, 128, 128] (Q/K dtype) with
        contiguous blocks, key_scale [num_blocks, 128] float32 per-token scales or None.
        Strides between blocks may exceed the block size (vLLM-style packed pages)."""
        torch = self.torch
        if keys.dtype != self.qk_torch_dtype or keys.dim() != 3 or tuple(keys.shape[1:]) != (BLOCK_TOKENS, INDEX_DIM):
            raise ValueError(f"index-K cache must be {self.qk_torch_dtype} [blocks, 128, 128]")
        if keys.stride(2) != 1 or keys.stride(1) != INDEX_DIM or keys.device != self.device:
            raise ValueError("index-K blocks must be contiguous and on the binding's device")
        if key_scale is not None:
            if key_scale.dtype != torch.float32 or key_scale.dim() != 2 or key_scale.shape[1] != BLOCK_TOKENS:
                raise ValueError("key scales must be float32 [blocks, 128]")
            if key_scale.shape[0] != keys.shape[0] or key_scale.stride(1) != 1 or key_scale.device != self.device:
                raise ValueError("key scales must match the index-K blocks and be contiguous per block")
        self.keys, self.key_scale = keys, key_scale
        return self

    def bind_query_inputs(self, inputs):
        """Read the packed decode queries of a vLLM-adapter QueryInputs in place of this
        binding's own buffers: query, weights, query scales and query ends become the
        inputs' tensors, which the adapter's `pack` and `bind_positions` fill every step
        (the reference binds the same persistent buffers as LI arguments 0, 2, 3 and its
        query ends, adapters/vllm/binding.py:65-85, selector.py:76-82). Needs fp8
        queries, bf16 weights, four rows per request and the inputs' batch and heads; call
        before the forward and the Index update are built. Requests then see
        min(seq_lens, query_ends) positions: seq_lens is set to the whole context."""
        if self.rows_per_request != 4 or self.batch != inputs.batch or self.heads != inputs.index_heads:
            raise ValueError("QueryInputs need a binding of four rows per request with their batch and heads")
        if self.qk_name != "fp8" or self.weight_code != abi.DTYPE_BF16 or self.query_ends is None:
            raise ValueError("QueryInputs need fp8 queries, bf16 weights and query ends")
        if self.query_scale is None or inputs.device != self.device:
            raise ValueError("QueryInputs need query scales on the binding's device")
        self.query, self.weights, self.query_scale = inputs.query, inputs.weights, inputs.scale
        self.query_ends = inputs.query_ends
        self.seq_lens.fill_(self.key_stride)
        self.query_inputs = inputs
        return self

    @property
    def num_blocks(self):
        return 0 if self.keys is None else int(self.keys.shape[0])

    def indexer_args(self):
        if self.keys is None:
            raise ValueError("bind_index_cache() must be called before the forward is built")
        p = abi.ptr
        elem = self.keys.element_size()
        return abi.IndexerArgs(
            query=p(self.query), weights=p(self.weights), query_scale=p(self.query_scale), keys=p(self.keys),
            key_scale=p(self.key_scale), block_table=p(self.block_table), seq_lens=p(self.seq_lens),
            query_ends=p(self.query_ends), score_keys=p(self.score_keys), histogram=p(self.histogram),
            status=p(self.status), key_block_stride=self.keys.stride(0) * elem,
            scale_block_stride=0 if self.key_scale is None else self.key_scale.stride(0),
            batch=self.batch, rows_per_request=self.rows_per_request, heads=self.heads, max_blocks=self.max_blocks,
            num_blocks=self.num_blocks, key_stride=self.key_stride, qk_dtype=self.qk_code,
            weight_dtype=self.weight_code,
        )

    def topk_args(self, use_histogram=True, split=True):
        """TopK arguments; with the scoring histogram the select runs on 4096-key segments
        (split=True) or one workgroup per row (split=False)."""
        p = abi.ptr
        return abi.TopkArgs(
            score_keys=p(self.score_keys), histogram=p(self.histogram) if use_histogram else 0,
            segments=p(self.topk_segments) if use_histogram and split else 0,
            seq_lens=p(self.seq_lens), query_ends=p(self.query_ends), topk=p(self.topk), status=p(self.status),
            batch=self.batch, rows_per_request=self.rows_per_request, key_stride=self.key_stride,
        )


class ContiguousFetch:
    """Fetch destination of the decode round: the selected KV rows of every query row,
    gathered from a paged HBM KV cache [num_blocks, 128, row_bytes] (uint8, rows
    contiguous inside a block) into `output` [rows, 2048, row_bytes].

    block_table defaults to the indexer's (index-K and KV pages share block ids, as in
    vLLM); pass another [batch, max_blocks] int32 table to decouple them."""

    def __init__(self, torch, rotating, kv_cache, *, block_table=None):
        if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 3 or kv_cache.shape[1] != BLOCK_TOKENS:
            raise ValueError("KV cache must be uint8 [blocks, 128, row_bytes]")
        row_bytes = int(kv_cache.shape[2])
        if row_bytes % 16 or kv_cache.stride(2) != 1 or kv_cache.stride(1) % 16 or kv_cache.stride(0) % 16:
            raise ValueError("KV rows must be contiguous multiples of 16 bytes")
        if kv_cache.device != rotating.device:
            raise ValueError("Fetch and LI must use the same device")
        table = rotating.block_table if block_table is None else block_table
        if table.dtype != torch.int32 or tuple(table.shape) != (rotating.batch, rotating.max_blocks):
            raise ValueError("Fetch block table must be int32 [batch, max_blocks]")
        self.torch, self.device = torch, rotating.device
        self.rotating, self.kv_cache, self.block_table = rotating, kv_cache, table
        self.row_bytes = row_bytes
        self.output = torch.zeros((rotating.rows, TOPK, row_bytes), dtype=torch.uint8, device=self.device)

    @property
    def logical_output(self):
        """Selected token ids per query row, [rows, 2048] (-1 = empty)."""
        return self.rotating.topk

    def fetch_args(self):
        p = abi.ptr
        r = self.rotating
        return abi.FetchArgs(
            topk=p(r.topk), kv_cache=p(self.kv_cache), block_table=p(self.block_table), output=p(self.output),
            status=p(r.status), kv_block_stride=self.kv_cache.stride(0), row_stride=self.kv_cache.stride(1),
            row_bytes=self.row_bytes, batch=r.batch, rows_per_request=r.rows_per_request, max_blocks=r.max_blocks,
            num_blocks=int(self.kv_cache.shape[0]),
        )
