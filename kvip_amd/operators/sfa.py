"""Sparse attention over the selected KV rows: `kvip_amd.sparse_attention` and the bound
`kvip_amd.SparseAttention`.

This is the consumer of the LIFetch outputs that the reference's service tests run on the
hot cache (tests/operators/lifetch/support/correctness.py:261-339, the C8 sparse flash
attention with 2048 sparse indices per query row, 656-byte rows of workloads.py:493-515):
per query row and head, softmax attention of a bf16 [576] query over the rows its indices
name, keys [nope * scale, rope], values nope * scale. The rows are read in place through a
block table, so the same launch serves the resident hot cache (indices = slot outputs,
`hot_cache_table`) and the gathered buffer of a contiguous Fetch (`gathered_table`).
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi

TOPK = 2048
BLOCK_TOKENS = 128
KEY_DIM = 576
VALUE_DIM = 512
ROW_BYTES = 656


class SparseAttention:
    """Output [rows, heads, 512] float32 and status allocated once; `bind` validates a call's
    tensors, `__call__` enqueues the launch on the current stream (graph-capturable)."""

    def __init__(self, torch, *, rows, heads, device, rows_per_request=1):
        if not 1 <= heads <= 128:
            raise ValueError("sparse attention supports 1..128 heads")
        if rows < 1 or rows % rows_per_request:
            raise ValueError("rows must be a positive multiple of rows_per_request")
        self.torch, self.device = torch, abi.device_of(torch, device)
        self.rows, self.heads, self.rows_per_request = rows, heads, rows_per_request
        self.output = torch.zeros((rows, heads, VALUE_DIM), dtype=torch.float32, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.library = abi.load_library()
        # Partials of the index splits (the launch splits each row's 2048 indices when there
        # are too few rows to fill the GPU).
        nbytes = int(self.library.kvip_hip_sparse_attention_workspace_bytes(rows, heads))
        self.workspace = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=self.device)
        self.args = None

    def bind(self, query, kv_cache, block_table, indices, scale=KEY_DIM ** -0.5):
        """query [rows, heads, 576] bf16; kv_cache uint8 [blocks, 128, row_stride] (or
        [blocks, 128, 1, row_stride]) with rows of 656 bytes; block_table int32
        [rows / rows_per_request, max_blocks]; indices int32 [rows, 2048] or
        [rows, 1, 2048], positions in the request's paged space (-1 = none)."""
        t = self.torch
        if query.dtype != t.bfloat16 or tuple(query.shape) != (self.rows, self.heads, KEY_DIM) or not query.is_contiguous():
            raise ValueError(f"query must be contiguous bfloat16 [{self.rows}, {self.heads}, 576]")
        if kv_cache.dim() == 4:
            kv_cache = kv_cache.view(kv_cache.shape[0], kv_cache.shape[1], kv_cache.shape[3])
        if (kv_cache.dtype not in (t.uint8, t.float8_e4m3fn) or kv_cache.dim() != 3 or kv_cache.shape[1] != BLOCK_TOKENS
                or kv_cache.shape[2] < ROW_BYTES or kv_cache.stride(2) != 1):
            raise ValueError("kv_cache must be 1-byte [blocks, 128, row_stride >= 656] with contiguous rows")
        batch = self.rows // self.rows_per_request
        if block_table.dtype != t.int32 or block_table.dim() != 2 or block_table.shape[0] != batch or \
                not block_table.is_contiguous():
            raise ValueError(f"block_table must be contiguous int32 [{batch}, max_blocks]")
        indices = indices.reshape(self.rows, -1) if indices.dim() == 3 else indices
        if indices.dtype != t.int32 or tuple(indices.shape) != (self.rows, TOPK) or not indices.is_contiguous():
            raise ValueError(f"indices must be contiguous int32 [{self.rows}, 2048]")
        for x in (query, kv_cache, block_table, indices):
            if x.device != self.device:
                raise ValueError("sparse attention tensors must share the output's device")
        p = abi.ptr
        self.args = abi.SparseAttnArgs(
            query=p(query), kv_cache=p(kv_cache), block_table=p(block_table), indices=p(indices),
            output=p(self.output), status=p(self.status), workspace=p(self.workspace),
            kv_block_stride=kv_cache.stride(0),
            row_stride=kv_cache.stride(1), rows=self.rows, rows_per_request=self.rows_per_request, heads=self.heads,
            max_blocks=int(block_table.shape[1]), num_blocks=int(kv_cache.shape[0]), scale=float(scale))
        self._bound = (query, kv_cache, block_table, indices)
        return self

    def __call__(self):
        if self.args is None:
            raise ValueError("bind() the sparse attention inputs first")
        abi.check(self.library.kvip_hip_sparse_attention(ctypes.byref(self.args),
                                                          abi.stream_handle(self.torch, self.device)),
                  "sparse attention")
        return self.output


def sparse_attention(query, kv_cache, block_table, indices, scale=KEY_DIM ** -0.5, *, rows_per_request=1):
    """One sparse-attention call (arguments as `SparseAttention.bind`); returns float32
    [rows, heads, 512]."""
    import torch

    op = SparseAttention(torch, rows=int(query.shape[0]), heads=int(query.shape[1]), device=query.device,
                         rows_per_request=rows_per_request)
    return op.bind(query, kv_cache, block_table, indices, scale)()


def hot_cache_table(torch, update):
    """Paged view of a ResidentIndexUpdate's hot cache for `sparse_attention`: returns
    (kv_cache [owners * hot_stride / 128, 128, row_bytes], block_table [batch,
    hot_stride / 128] int32 with block_table[b][j] = row_owners[b] * hot_stride / 128 + j);
    slot outputs are then the indices. The table reads row_owners when called."""
    owners, stride, row = (int(x) for x in update.hot_cache.shape)
    if stride % BLOCK_TOKENS:
        raise ValueError("the hot cache's rows per owner must be a multiple of 128")
    per_owner = stride // BLOCK_TOKENS
    kv = update.hot_cache.view(owners * per_owner, BLOCK_TOKENS, row)
    offsets = torch.arange(per_owner, dtype=torch.int32, device=update.hot_cache.device)
    table = (update.row_owners.to(torch.int32)[:, None] * per_owner + offsets[None, :]).contiguous()
    return kv, table


def gathered_table(torch, update):
    """Paged view of a ContiguousFetch output [rows, 2048, row_bytes] for `sparse_attention`
    with one query row per request: (kv_cache [rows * 16, 128, row_bytes], block_table
    [rows, 16] int32, indices [rows, 2048] int32 = the rank, -1 where TopK was empty)."""
    out = update.output
    rows, _, row = (int(x) for x in out.shape)
    kv = out.view(rows * (TOPK // BLOCK_TOKENS), BLOCK_TOKENS, row)
    table = (torch.arange(rows, dtype=torch.int32, device=out.device)[:, None] * (TOPK // BLOCK_TOKENS) +
             torch.arange(TOPK // BLOCK_TOKENS, dtype=torch.int32, device=out.device)[None, :]).contiguous()
    rank = torch.arange(TOPK, dtype=torch.int32, device=out.device)[None, :].expand(rows, TOPK)
    indices = torch.where(update.rotating.topk >= 0, rank, torch.full_like(rank, -1)).contiguous()
    return kv, table, indices
