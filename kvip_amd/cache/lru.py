"""`kvip_amd.SlotLRU`: the resident-slot LRU on the device (python/kvip/cache/lru.py:14-118).

Same lifecycle as the reference: `resize(capacity, committed)` grows storage and appends
newly committed slots at the most-recent end (or resets to a cold ascending chain when the
committed prefix shrinks or starts); `commit(destinations)` moves the unique destination
slots below `active` to the most-recent end in ascending slot-id order. After each call
`slots` ([1, 2048] int32) holds the min(2048, active) least recently used slots, oldest
first, -1 padded, and `bitmap` ([1, words] int32, words rounded up to a multiple of 8) their
membership bits. State lives on the device as the LRU order array, so `commit` takes a
device tensor and enqueues on the current stream without a host sync (graph-capturable).
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi

TOPK = 2048
BITMAP_WORD_BITS = 32
BITMAP_ALIGNMENT_WORDS = 8
MAX_SLOTS = (1 << 17) + 20 * 128


class SlotLRU:
    def __init__(self, device="cuda"):
        import torch

        self.torch, self.device = torch, abi.device_of(torch, device)
        self.version = 0
        self.active = 0
        self.capacity = 0
        self.order = torch.empty(0, dtype=torch.int32, device=self.device)
        self.scratch = torch.empty(0, dtype=torch.int32, device=self.device)
        self.slots = torch.full((1, TOPK), -1, dtype=torch.int32, device=self.device)
        self.bitmap = torch.zeros((1, 0), dtype=torch.int32, device=self.device)
        self._args = None

    def _bind(self):
        self._args = abi.LruArgs(order=abi.ptr(self.order), scratch=abi.ptr(self.scratch),
                                 slots=abi.ptr(self.slots), bitmap=abi.ptr(self.bitmap),
                                 capacity=self.capacity, bitmap_words=self.bitmap.shape[1])

    def _stream(self):
        return abi.stream_handle(self.torch, self.device)

    def resize(self, capacity, committed):
        """Grow storage and append newly committed slots, preserving LRU order (lru.py:33-83)."""
        if not 0 <= committed <= capacity:
            raise ValueError("Committed slots must fit HBM capacity")
        torch = self.torch
        changed = False
        if capacity > self.capacity:
            capacity = max(capacity, 2 * self.capacity)
            if capacity > MAX_SLOTS:
                raise ValueError(f"SlotLRU capacity above {MAX_SLOTS} slots")
            order = torch.full((capacity,), -1, dtype=torch.int32, device=self.device)
            order[: self.capacity].copy_(self.order)
            self.order = order
            self.scratch = torch.empty(capacity, dtype=torch.int32, device=self.device)
            words = (capacity + BITMAP_WORD_BITS - 1) // BITMAP_WORD_BITS
            words = (words + BITMAP_ALIGNMENT_WORDS - 1) // BITMAP_ALIGNMENT_WORDS * BITMAP_ALIGNMENT_WORDS
            self.bitmap = torch.zeros((1, words), dtype=torch.int32, device=self.device)
            self.capacity = capacity
            self._bind()
            changed = True
        lib = abi.load_library()
        if committed < self.active or self.active == 0 < committed:
            abi.check(lib.kvip_hip_lru_reset(ctypes.byref(self._args), committed, self._stream()), "SlotLRU reset")
            self.active = committed
            self.version += 1
            return
        if committed > self.active:
            abi.check(lib.kvip_hip_lru_extend(ctypes.byref(self._args), self.active, committed, self._stream()),
                      "SlotLRU extend")
            self.active = committed
            changed = True
        elif changed:
            abi.check(lib.kvip_hip_lru_commit(ctypes.byref(self._args), None, 0, self.active, self._stream()),
                      "SlotLRU victims")
        if changed:
            self.version += 1

    def commit(self, destinations):
        """Consume the accessed slots (a device int32 tensor); slots outside [0, active) are
        ignored, as ABC hits do not enter the chain (lru.py:96-118)."""
        torch = self.torch
        if self.active == 0:
            return
        if not isinstance(destinations, torch.Tensor) or destinations.device != self.device \
                or destinations.dtype != torch.int32 or not destinations.is_contiguous():
            raise ValueError("SlotLRU.commit takes a contiguous int32 tensor on the LRU's device")
        lib = abi.load_library()
        abi.check(lib.kvip_hip_lru_commit(ctypes.byref(self._args), abi.ptr(destinations), destinations.numel(),
                                          self.active, self._stream()), "SlotLRU commit")
        self.version += 1
