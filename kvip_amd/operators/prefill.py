"""Prefill lightning indexer with TopK-2048: `kvip_amd.PrefillIndexer` and the functional
`kvip_amd.quant_lightning_indexer`.

The reference's vLLM selector runs prefill rows (and the prefill part of mixed batches)
through the native quantised lightning indexer (python/kvip/adapters/vllm/selector.py:
126-154, torch_npu.npu_quant_lightning_indexer with layout TND and sparse_mode 3, as
called in tests/operators/lifetch/support/execution.py:126-145). This module is that
surface on MI355X: packed query rows of several sequences (cumulative query lengths)
against their paged index-K, right-down causal, fp8 e4m3 or bf16 Q/K (the bf16 form is the
unquantised lightning indexer of the same selector path), per-row TopK-2048 of positions
within each sequence (-1 padded), tie-broken to the lower position as in decode.

`PrefillIndexer` allocates its buffers once (rows and context bounds fixed at
construction) and only enqueues on the current stream when called, so a bound call can
be captured into a hipGraph. `quant_lightning_indexer` builds one for a single call.
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi

TOPK = 2048
BLOCK_TOKENS = 128
INDEX_DIM = 128
MAX_SEQUENCES = 1024


class PrefillIndexer:
    def __init__(self, torch, *, max_rows, max_context, max_sequences, device, heads=64, weight_dtype=None):
        if heads not in (32, 64):
            raise ValueError("prefill LI supports 32 or 64 heads")
        if not 1 <= max_sequences <= MAX_SEQUENCES:
            raise ValueError(f"max_sequences must be in 1..{MAX_SEQUENCES}")
        weight_dtype = torch.float32 if weight_dtype is None else weight_dtype
        if weight_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("weights must be float32 or bfloat16")
        self.torch, self.device = torch, abi.device_of(torch, device)
        self.heads, self.max_rows, self.max_sequences = heads, max_rows, max_sequences
        self.max_blocks = (max_context + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        self.key_stride = self.max_blocks * BLOCK_TOKENS
        self.weight_code = abi.DTYPE_FP32 if weight_dtype == torch.float32 else abi.DTYPE_BF16
        self.weight_dtype = weight_dtype
        dev = self.device
        self.score_keys = torch.zeros((max_rows, self.key_stride), dtype=torch.int16, device=dev)
        self.histogram = torch.zeros((max_rows, 256), dtype=torch.int32, device=dev)
        self.row_valid = torch.zeros(max_rows, dtype=torch.int32, device=dev)
        self.topk = torch.full((max_rows, TOPK), -1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.library = abi.load_library()
        # Scoring grid: 0 = one workgroup per work unit (8 query rows x 4096 key positions);
        # n > 0 = at most n workgroups striding over the units (kvip_hip_indexer_prefill_grid),
        # for rounds that run other kernels beside the prefill.
        self.workgroups = 0

    def __call__(self, query, weights, query_scale, key, key_scale, cu_seqlens_q, seq_lens_k, block_table):
        """query [rows, heads, 128] fp8 e4m3 or bf16; weights [rows, heads]; query_scale
        [rows, heads] float32 or None; key [blocks, 128, 128] of the query's dtype
        (contiguous blocks); key_scale
        [blocks, 128] float32 or None; cu_seqlens_q [sequences + 1] int32 (device);
        seq_lens_k [sequences] int32; block_table [sequences, max_blocks] int32. Returns the
        TopK view [rows, 2048] int32 (positions within each row's sequence)."""
        self.bind(query, weights, query_scale, key, key_scale, cu_seqlens_q, seq_lens_k, block_table)
        self.score()
        return self.select()

    def bind(self, query, weights, query_scale, key, key_scale, cu_seqlens_q, seq_lens_k, block_table):
        """Validate one call's tensors (same meaning as __call__) and keep their launch
        arguments; `score()` and `select()` then enqueue the two launches."""
        t = self.torch
        rows, sequences = int(query.shape[0]), int(seq_lens_k.shape[0])
        if not 1 <= rows <= self.max_rows or not 1 <= sequences <= self.max_sequences:
            raise ValueError("rows / sequences exceed the bound sizes")
        if query.dtype not in (t.float8_e4m3fn, t.bfloat16) or tuple(query.shape[1:]) != (self.heads, INDEX_DIM):
            raise ValueError(f"query must be float8_e4m3fn or bfloat16 [rows, {self.heads}, 128]")
        if not query.is_contiguous():
            raise ValueError("query must be contiguous")
        if weights.dtype != self.weight_dtype or tuple(weights.shape) != (rows, self.heads):
            raise ValueError("weights must match the bound dtype and [rows, heads]")
        if query_scale is not None and (query_scale.dtype != t.float32 or tuple(query_scale.shape) != (rows, self.heads)):
            raise ValueError("query_scale must be float32 [rows, heads]")
        if key.dtype != query.dtype or key.dim() != 3 or tuple(key.shape[1:]) != (BLOCK_TOKENS, INDEX_DIM):
            raise ValueError(f"key must be {query.dtype} [blocks, 128, 128] (the query's dtype)")
        if key.stride(2) != 1 or key.stride(1) != INDEX_DIM:
            raise ValueError("index-K blocks must be contiguous")
        if key_scale is not None and (key_scale.dtype != t.float32 or key_scale.dim() != 2 or
                                      key_scale.shape[0] != key.shape[0] or key_scale.stride(1) != 1):
            raise ValueError("key_scale must be float32 [blocks, 128]")
        if block_table.dtype != t.int32 or block_table.dim() != 2 or block_table.shape[0] != sequences:
            raise ValueError("block_table must be int32 [sequences, blocks]")
        if block_table.shape[1] > self.max_blocks or not block_table.is_contiguous():
            raise ValueError("block_table exceeds the bound context or is not contiguous")
        for x in (cu_seqlens_q, seq_lens_k):
            if x.dtype != t.int32 or not x.is_contiguous():
                raise ValueError("sequence lengths must be contiguous int32")
        if cu_seqlens_q.shape[0] != sequences + 1:
            raise ValueError("cu_seqlens_q must have sequences + 1 entries")
        p = abi.ptr
        args = abi.PrefillArgs(
            query=p(query), weights=p(weights), query_scale=p(query_scale), keys=p(key), key_scale=p(key_scale),
            block_table=p(block_table), cu_seqlens_q=p(cu_seqlens_q), seq_lens_k=p(seq_lens_k),
            score_keys=p(self.score_keys), histogram=p(self.histogram), row_valid=p(self.row_valid),
            status=p(self.status), key_block_stride=key.stride(0) * key.element_size(), scale_block_stride=0 if key_scale is None
            else key_scale.stride(0), sequences=sequences, rows=rows, heads=self.heads,
            max_blocks=int(block_table.shape[1]), num_blocks=int(key.shape[0]), key_stride=self.key_stride,
            qk_dtype=abi.DTYPE_FP8_E4M3 if query.dtype == t.float8_e4m3fn else abi.DTYPE_BF16,
            weight_dtype=self.weight_code)
        topk = abi.TopkArgs(score_keys=p(self.score_keys), histogram=p(self.histogram), segments=0,
                            seq_lens=p(self.row_valid), query_ends=0, topk=p(self.topk), status=p(self.status),
                            batch=rows, rows_per_request=1, key_stride=self.key_stride)
        # The bound tensors stay referenced for as long as their pointers are kept.
        self._bound = (query, weights, query_scale, key, key_scale, cu_seqlens_q, seq_lens_k, block_table)
        self._args, self._topk_args, self._rows = args, topk, rows

    def score(self, workgroups=None):
        """Scoring launch: score keys, per-row visible lengths and high-byte histograms.
        workgroups: grid bound for this launch (None: self.workgroups)."""
        stream = abi.stream_handle(self.torch, self.device)
        workgroups = self.workgroups if workgroups is None else int(workgroups)
        if workgroups < 0:
            raise ValueError("workgroups must be >= 0")
        if workgroups:
            abi.check(self.library.kvip_hip_indexer_prefill_grid(ctypes.byref(self._args), workgroups, stream),
                      "prefill LI")
        else:
            abi.check(self.library.kvip_hip_indexer_prefill(ctypes.byref(self._args), stream), "prefill LI")

    def select(self):
        """TopK-2048 launch over the scored rows (consumes and re-zeroes the histograms)."""
        abi.check(self.library.kvip_hip_topk(ctypes.byref(self._topk_args),
                                             abi.stream_handle(self.torch, self.device)), "prefill TopK")
        return self.topk[:self._rows]


def quant_lightning_indexer(query, key, weights, query_dequant_scale, key_dequant_scale, actual_seq_lengths_query,
                            actual_seq_lengths_key, block_table, *, query_quant_mode=0, key_quant_mode=0,
                            layout_query="TND", layout_key="PA_BSND", sparse_count=2048, sparse_mode=3):
    """One prefill selection with the argument names of the native indexer call
    (execution.py:126-145): TND query rows with cumulative `actual_seq_lengths_query`,
    paged keys [blocks, 128, 1, 128] or [blocks, 128, 128], per-sequence key lengths,
    right-down causal (sparse_mode 3). Returns int32 [rows, 1, 2048]."""
    import torch

    if layout_query != "TND" or layout_key != "PA_BSND" or sparse_mode != 3 or sparse_count != TOPK:
        raise ValueError("supported: layout_query TND, layout_key PA_BSND, sparse_mode 3, sparse_count 2048")
    if query_quant_mode != 0 or key_quant_mode != 0:
        raise ValueError("supported quant modes: 0 (per-row dequant scales)")
    if key.dim() == 4:
        key = key.view(key.shape[0], key.shape[1], key.shape[3])
    if key_dequant_scale is not None and key_dequant_scale.dim() == 3:
        key_dequant_scale = key_dequant_scale.view(key_dequant_scale.shape[0], key_dequant_scale.shape[1])
    heads = int(query.shape[-2])
    q = query.view(-1, heads, INDEX_DIM)
    cu = torch.cat([torch.zeros(1, dtype=torch.int32, device=q.device), actual_seq_lengths_query.int()]).contiguous()
    ctx = int(block_table.shape[1]) * BLOCK_TOKENS
    idx = PrefillIndexer(torch, max_rows=int(q.shape[0]), max_context=ctx, max_sequences=int(block_table.shape[0]),
                         device=q.device, heads=heads, weight_dtype=weights.dtype)
    qs = None if query_dequant_scale is None else query_dequant_scale.view(q.shape[0], heads).float().contiguous()
    out = idx(q, weights.view(q.shape[0], heads).contiguous(), qs, key, key_dequant_scale, cu,
              actual_seq_lengths_key.int().contiguous(), block_table.int().contiguous())
    return out.view(-1, 1, TOPK)
