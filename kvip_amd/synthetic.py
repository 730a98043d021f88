"""Seeded synthetic decode workloads at the benchmark shapes (no datasets, no network).

`decode_workload` builds, directly on the device, everything one LIFetch decode round
reads: request context lengths, a shuffled block table, a paged index-K cache with
per-token scales, the index queries and head weights, and a paged KV cache of
656-byte rows filled with random bytes (any misplaced byte is detectable).

Configurations:
  c1: batch 4, ctx 4096, bf16 Q/K ~N(0,1), fp32 weights ~N(0,1)/8, no scales.
  c2: batch 64, ctx ~U{8192..32768}, fp8 e4m3 Q/K from N(0,1) (saturating cast),
      per-token key scale ~U(0.5, 2), fp32 weights ~N(0,1)/8, KV rows of 656 bytes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

BLOCK_TOKENS = 128
INDEX_DIM = 128


@dataclass
class DecodeWorkload:
    ctx: np.ndarray            # [batch] context tokens per request
    block_table: object        # torch int32 [batch, max_blocks]
    keys: object               # torch [num_blocks, 128, 128] fp8 e4m3 / bf16
    key_scale: object          # torch float32 [num_blocks, 128] or None
    query: object              # torch [rows, heads, 128]
    weights: object            # torch [rows, heads]
    query_scale: object        # torch float32 [rows, heads] or None
    kv_cache: object           # torch uint8 [num_blocks, 128, row_bytes] or None
    rows_per_request: int
    seed: int

    @property
    def batch(self):
        return len(self.ctx)

    @property
    def max_blocks(self):
        return int(self.block_table.shape[1])


def saturating_fp8(torch, x):
    return x.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def decode_workload(torch, *, batch, device, ctx=None, ctx_low=None, ctx_high=None, heads=64, qk="fp8",
                    weight_dtype=None, key_scale=True, query_scale=False, rows_per_request=1,
                    kv_row_bytes=656, seed=0, max_context=None):
    rng = np.random.default_rng(seed)
    if ctx is None:
        ctx = rng.integers(ctx_low, ctx_high + 1, size=batch)
    ctx = np.asarray(ctx, dtype=np.int64)
    blocks_per = (ctx + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    max_ctx = int(max_context or max(int(ctx.max()), 1))
    max_blocks = (max_ctx + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    num_blocks = max(int(blocks_per.sum()), 1)
    perm = rng.permutation(num_blocks).astype(np.int32)
    table = np.zeros((batch, max_blocks), np.int32)
    offset = 0
    for b, n in enumerate(blocks_per):
        table[b, :n] = perm[offset:offset + n]
        offset += n
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dev = torch.device(device)
    rows = batch * rows_per_request
    weight_dtype = torch.float32 if weight_dtype is None else weight_dtype

    def normal(shape):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)

    if qk == "fp8":
        keys = saturating_fp8(torch, normal((num_blocks, BLOCK_TOKENS, INDEX_DIM)))
        query = saturating_fp8(torch, normal((rows, heads, INDEX_DIM)))
    else:
        keys = normal((num_blocks, BLOCK_TOKENS, INDEX_DIM)).to(torch.bfloat16)
        query = normal((rows, heads, INDEX_DIM)).to(torch.bfloat16)
    weights = (normal((rows, heads)) / 8).to(weight_dtype)
    ks = None
    if key_scale:
        ks = torch.rand((num_blocks, BLOCK_TOKENS), generator=gen, device=dev, dtype=torch.float32) * 1.5 + 0.5
    qs = None
    if query_scale:
        qs = torch.rand((rows, heads), generator=gen, device=dev, dtype=torch.float32) + 0.5
    kv = None
    if kv_row_bytes:
        kv = torch.randint(0, 256, (num_blocks, BLOCK_TOKENS, kv_row_bytes), generator=gen, device=dev,
                           dtype=torch.uint8)
    return DecodeWorkload(ctx=ctx, block_table=torch.from_numpy(table).to(dev), keys=keys, key_scale=ks,
                          query=query, weights=weights, query_scale=qs, kv_cache=kv,
                          rows_per_request=rows_per_request, seed=seed)


def config_workload(torch, name, device, seed=2026):
    """The benchmark configurations by name ('c1' or 'c2')."""
    if name == "c1":
        return decode_workload(torch, batch=4, ctx=[4096] * 4, device=device, qk="bf16", key_scale=False,
                               seed=seed)
    if name == "c2":
        return decode_workload(torch, batch=64, ctx_low=8192, ctx_high=32768, device=device, qk="fp8",
                               key_scale=True, seed=seed, max_context=32768)
    raise ValueError(f"unknown decode configuration {name!r}")


def bind(torch, kvip, wl, *, query_ends=None):
    """LIFetchBinding + ContiguousFetch + LIFetch forward for a workload."""
    heads = int(wl.query.shape[1])
    qk = "fp8" if wl.query.dtype == torch.float8_e4m3fn else "bf16"
    rot = kvip.LIFetchBinding(torch, batch=wl.batch, max_context=wl.max_blocks * BLOCK_TOKENS,
                              device=wl.query.device, heads=heads, rows_per_request=wl.rows_per_request,
                              qk_dtype=qk, weight_dtype=wl.weights.dtype, query_scale=wl.query_scale is not None,
                              query_ends=query_ends is not None)
    rot.query.copy_(wl.query)
    rot.weights.copy_(wl.weights)
    if wl.query_scale is not None:
        rot.query_scale.copy_(wl.query_scale)
    rot.seq_lens.copy_(torch.from_numpy(wl.ctx.astype(np.int32)))
    if query_ends is not None:
        rot.query_ends.copy_(torch.as_tensor(np.asarray(query_ends, np.int32)))
    rot.block_table.copy_(wl.block_table)
    rot.bind_index_cache(wl.keys, wl.key_scale)
    upd = kvip.ContiguousFetch(torch, rot, wl.kv_cache)
    return rot, upd, kvip.LIFetch(rot, upd)
