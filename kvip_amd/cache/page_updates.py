"""Publication of appended KV pages across all requests and groups in one upload and one
launch: `PageUpdates`, mirroring the reference's (python/kvip/cache/page_updates.py:5-62)
constructor, `nbytes` and `submit(rows, ring)`. Rows are {flat page index, page address,
old map offset or -1}; the launch is `kvip_hip_publish_pages`. There is no CPU path: the
tables must be GPU tensors."""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi


class PageUpdates:
    def __init__(self, torch, addresses, valid, token_to_slot, *, fused=(), widths=(), token_bytes=656,
                 block_size=128):
        """addresses int64 [owners, groups, pages], valid uint8 of the same shape,
        token_to_slot int32 (the ABC map), fused: per group an int64 [owners, history]
        token-address table with `widths[group]` tokens of `token_bytes` per position."""
        if addresses.dim() != 3 or addresses.dtype != torch.int64 or not addresses.is_contiguous():
            raise ValueError("page addresses must be contiguous int64 [owners, groups, pages]")
        if valid.shape != addresses.shape or valid.dtype != torch.uint8 or not valid.is_contiguous():
            raise ValueError("page validity must be contiguous uint8 shaped like the addresses")
        if token_to_slot.dtype != torch.int32 or not token_to_slot.is_contiguous():
            raise ValueError("token_to_slot must be contiguous int32")
        if len(fused) != len(widths) or (fused and len(fused) != addresses.shape[1]):
            raise ValueError("fused tables need one table and one width per group")
        for t in fused:
            if t.dtype != torch.int64 or t.dim() != 2 or not t.is_contiguous() or t.shape != fused[0].shape or \
                    t.shape[0] != addresses.shape[0]:
                raise ValueError("fused tables must be contiguous int64 [owners, history] of one shape")
        if not 1 <= block_size <= 256:
            raise ValueError("block_size must be in 1..256")
        self.torch = torch
        self.addresses, self.valid, self.token_to_slot = addresses, valid, token_to_slot
        self.block_size = block_size
        self.fused = tuple(fused)
        self.widths, self.token_bytes = tuple(widths), token_bytes
        dev = addresses.device
        if dev.type != "cuda" or any(t.device != dev for t in (valid, token_to_slot, *self.fused)):
            raise ValueError("page tables must be GPU tensors on one device (kvip_amd has no CPU path)")
        shape = (addresses.numel(), 3)
        self.device = torch.empty(shape, dtype=torch.int64, device=dev)
        self.host = [torch.empty(shape, dtype=torch.int64, pin_memory=True) for _ in range(2)]
        self.fused_table = torch.tensor(
            [(t.data_ptr(), w * token_bytes) for t, w in zip(self.fused, self.widths)] or [(0, 0)],
            dtype=torch.int64, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.events = [None, None]  # completion of the last copy out of each staging buffer
        self.library = abi.load_library()

    @property
    def nbytes(self):
        return self.device.numel() * self.device.element_size() + self.fused_table.numel() * 8

    def submit(self, rows, ring):
        """rows: sequence of (flat page index, address, clear offset or -1); ring selects the
        pinned staging buffer (alternate it between steps so a pending copy is never
        overwritten; a buffer whose previous copy is still pending is waited for)."""
        if not rows:
            return
        count = len(rows)
        if count > self.device.shape[0]:
            raise ValueError("more page rows than page entries")
        torch = self.torch
        if self.events[ring] is not None:
            self.events[ring].synchronize()
        host = self.host[ring][:count]
        host.numpy()[:] = rows
        self.device[:count].copy_(host, non_blocking=True)
        if self.events[ring] is None:
            self.events[ring] = torch.cuda.Event()
        self.events[ring].record(torch.cuda.current_stream(self.addresses.device))
        p = abi.ptr
        a = self.addresses
        args = abi.PageArgs(
            rows=p(self.device), addresses=p(a), valid=p(self.valid), token_to_slot=p(self.token_to_slot),
            fused=p(self.fused_table) if self.fused else 0, status=p(self.status), entries=a.numel(),
            map_entries=self.token_to_slot.numel(), count=count, groups=int(a.shape[1]), pages=int(a.shape[2]),
            block_size=self.block_size, history=int(self.fused[0].shape[1]) if self.fused else 0)
        abi.check(self.library.kvip_hip_publish_pages(ctypes.byref(args), abi.stream_handle(self.torch, a.device)),
                  "publish pages")
