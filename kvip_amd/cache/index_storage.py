"""Persistent Index rows of every owner, on the device.

Interface of the reference's IndexCacheStorage (python/kvip/cache/index_storage.py:9-71):
the tables `keys` uint8 [owners, history, 128], `scales` float32 [owners, history],
`addresses` int64 [owners, history] (the committed KV address of each position),
`logical_ids` int64 [owners, history] and `hot_valid` int32 [owners, resident]; `prepare`
resets the metadata of owners that a new request takes over, `publish` appends the
per-token addresses of newly committed pages and never rewrites an entry published
earlier (the Index update may have permuted it since).

Layout: the five tables are views into one device arena, each starting on a 256-byte
boundary, so the whole storage is a single HBM allocation made once. The owner lifecycle
is one record per owner; the owners a step recycles are reset together, with one device
operation per table.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np

from kvip_amd.runtime import abi

INDEX_DIM = 128
ARENA_ALIGN = 256


@dataclass
class OwnerRecord:
    """Lifecycle of one owner row: the request holding it, whether that request's restored
    prefix has been read into the Index, and how many pages of addresses are published."""
    request: Any = None
    prefix_imported: bool = False
    pages: int = 0


class IndexCacheStorage:
    def __init__(self, torch, owners, history, resident, device):
        if owners < 1 or history < 1 or not 0 <= resident <= history:
            raise ValueError(f"Index storage needs owners >= 1 and 0 <= resident <= history "
                             f"(got {owners}, {history}, {resident})")
        self.torch, self.history, self.device = torch, int(history), abi.device_of(torch, device)
        self.owners, self.resident = int(owners), int(resident)
        tables = (("keys", torch.uint8, (owners, history, INDEX_DIM)),
                  ("scales", torch.float32, (owners, history)),
                  ("addresses", torch.int64, (owners, history)),
                  ("logical_ids", torch.int64, (owners, history)),
                  ("hot_valid", torch.int32, (owners, resident)))
        spans, end = [], 0
        for name, dtype, shape in tables:
            size = int(np.prod(shape)) * torch.empty(0, dtype=dtype).element_size()
            spans.append((name, dtype, shape, end, size))
            end = (end + size + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
        self._arena = torch.empty(max(end, ARENA_ALIGN), dtype=torch.uint8, device=self.device)
        for name, dtype, shape, offset, size in spans:
            setattr(self, name, self._arena[offset:offset + size].view(dtype).view(shape))
        self.positions = torch.arange(history, dtype=torch.int64, device=self.device)
        self.keys.zero_()
        self.scales.fill_(1.0)
        self.addresses.zero_()
        self.logical_ids.copy_(self.positions.expand(owners, -1))
        self.hot_valid.zero_()
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.records = {}

    @property
    def nbytes(self):
        """Device bytes held by the storage (the arena and the position ramp)."""
        return self._arena.numel() + self.positions.numel() * self.positions.element_size()

    @property
    def imported(self):
        """Owners whose current request's restored prefix is already in the Index."""
        return {o for o, r in self.records.items() if r.prefix_imported}

    def record(self, owner):
        return self.records.setdefault(int(owner), OwnerRecord())

    def prepare(self, plans):
        """Before a step is queued: every owner whose plan names a request other than the
        one it holds starts over (logical ids back to positions, no residency, no published
        addresses). All such owners of the step are reset together."""
        fresh = []
        for plan in plans:
            rec = self.record(plan.owner)
            if rec.request == plan.request:
                continue
            self.records[int(plan.owner)] = OwnerRecord(request=plan.request)
            fresh.append(int(plan.owner))
        if not fresh:
            return
        torch = self.torch
        rows = torch.tensor(sorted(set(fresh)), dtype=torch.int64, device=self.device)
        self.logical_ids.index_copy_(0, rows, self.positions.expand(rows.numel(), -1))
        self.hot_valid.index_fill_(0, rows, 0)
        self.addresses.index_fill_(0, rows, 0)

    def publish(self, owner, page_addresses, *, block_size, token_bytes):
        """Append the per-token addresses of the pages committed since the last call:
        position p of page j gets page_addresses[j] + (p % block_size) * token_bytes. The
        page list may only grow, and only up to the bound history."""
        rec = self.record(owner)
        count = len(page_addresses)
        if count < rec.pages:
            raise ValueError(f"owner {owner}: {count} committed pages, fewer than the {rec.pages} already published")
        if count * block_size > self.history:
            raise ValueError(f"owner {owner}: {count} pages of {block_size} tokens exceed the bound history "
                             f"{self.history}")
        if count == rec.pages:
            return
        new = np.asarray(page_addresses[rec.pages:], dtype=np.int64)
        per_token = (new[:, None] + np.arange(block_size, dtype=np.int64)[None, :] * int(token_bytes)).reshape(-1)
        first = rec.pages * block_size
        self.addresses[int(owner), first:first + per_token.size].copy_(self.torch.from_numpy(per_token))
        rec.pages = count
