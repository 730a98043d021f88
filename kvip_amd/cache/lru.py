"""`kvip_amd.SlotLRU`: the resident-slot LRU on the device (python/kvip/cache/lru.py:14-118).

Same lifecycle as the reference: `resize(capacity, committed)` grows storage and appends
newly committed slots at the most-recent end (or resets to a cold ascending chain when the
committed prefix shrinks or starts); `commit(destinations)` moves the unique destination
slots below `active` to the most-recent end in ascending slot-id order. After each call
`slots` ([1, 2048] int32) holds the min(2048, active) least recently used slots, oldest
first, -1 padded, and `bitmap` ([1, words] int32, words rounded up to a multiple of 8) their
membership bits. State lives on the device as the LRU order array: `commit` of a device
int32 tensor enqueues on the current stream without a host sync (graph-capturable); host
arrays (the reference's numpy call) are copied to the device first.
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
            raise ValueError(f"cannot commit {committed} slots into a capacity of {capacity}")
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
        """Consume the accessed slots; slots outside [0, active) are ignored, as ABC hits do
        not enter the chain (lru.py:96-118). `destinations` is a contiguous int32 tensor on
        the LRU's device (enqueued without a host sync, graph-capturable) or, as the
        reference takes it, any integer array or tensor elsewhere, which is first copied to
        the device as int32 (a blocking copy)."""
        torch = self.torch
        if self.active == 0:
            return
        if not isinstance(destinations, torch.Tensor):
            import numpy as np

            arr = np.asarray(destinations)
            if arr.dtype.kind not in "iu":
                raise ValueError("SlotLRU.commit takes integer slot ids")
            destinations = torch.from_numpy(np.ascontiguousarray(arr.reshape(-1), dtype=np.int32))
        elif destinations.dtype.is_floating_point or destinations.dtype.is_complex or destinations.dtype == torch.bool:
            raise ValueError("SlotLRU.commit takes integer slot ids")
        if destinations.device != self.device or destinations.dtype != torch.int32 or not destinations.is_contiguous():
            destinations = destinations.reshape(-1).to(device=self.device, dtype=torch.int32).contiguous()
        lib = abi.load_library()
        abi.check(lib.kvip_hip_lru_commit(ctypes.byref(self._args), abi.ptr(destinations), destinations.numel(),
                                          self.active, self._stream()), "SlotLRU commit")
        self.version += 1


class SlotLRUChains:
    """The slot LRUs of a whole batch, one chain per request, as one set of device arrays
    (no reference counterpart: the reference holds one SlotLRU per request and commits
    each from the host). Every chain has the same fixed `capacity` and evicts among the
    committed slots [0, active). `slots` [chains, 2048] holds every chain's victim
    candidates, oldest first, -1 padded; it may be a caller's buffer (for instance a
    ResidentIndexUpdate's `lru_slots`), so that a commit refreshes the next round's
    candidates in place. `commit(destinations)` takes int32 [chains, count] (a row per
    chain; slots outside [0, active), such as -1 padding, are ignored) and is one launch
    for the whole batch, enqueued on the current stream: a serving round can commit inside
    its captured hipGraph."""

    def __init__(self, torch, chains, capacity, device, *, active=None, slots=None):
        if not 1 <= chains <= 65535:
            raise ValueError(f"chains must be in 1..65535 (got {chains})")
        if not 1 <= capacity <= MAX_SLOTS:
            raise ValueError(f"capacity must be in 1..{MAX_SLOTS} (got {capacity})")
        self.torch, self.device = torch, abi.device_of(torch, device)
        self.chains, self.capacity = int(chains), int(capacity)
        words = (capacity + BITMAP_WORD_BITS - 1) // BITMAP_WORD_BITS
        words = (words + BITMAP_ALIGNMENT_WORDS - 1) // BITMAP_ALIGNMENT_WORDS * BITMAP_ALIGNMENT_WORDS
        dev = self.device
        self.order = torch.full((chains, capacity), -1, dtype=torch.int32, device=dev)
        self.scratch = torch.empty((chains, capacity), dtype=torch.int32, device=dev)
        self.bitmap = torch.zeros((chains, words), dtype=torch.int32, device=dev)
        if slots is None:
            slots = torch.full((chains, TOPK), -1, dtype=torch.int32, device=dev)
        if (tuple(slots.shape) != (chains, TOPK) or slots.dtype != torch.int32 or not slots.is_contiguous()
                or slots.device != dev):
            raise ValueError(f"slots must be a contiguous int32 [{chains}, {TOPK}] tensor on {dev}")
        self.slots = slots
        self._args = abi.LruArgs(order=abi.ptr(self.order), scratch=abi.ptr(self.scratch), slots=abi.ptr(slots),
                                 bitmap=abi.ptr(self.bitmap), capacity=self.capacity, bitmap_words=words)
        self.library = abi.load_library()
        self.active = 0
        self.reset(self.capacity if active is None else active)

    def _stream(self):
        return abi.stream_handle(self.torch, self.device)

    def reset(self, active):
        """Every chain becomes a cold LRU of the slots [0, active) in ascending order."""
        if not 0 <= active <= self.capacity:
            raise ValueError(f"active must be in 0..{self.capacity} (got {active})")
        abi.check(self.library.kvip_hip_lru_reset_chains(ctypes.byref(self._args), self.chains, int(active),
                                                         self._stream()), "SlotLRUChains reset")
        self.active = int(active)

    def commit(self, destinations):
        """Move each chain's accessed slots (row c of `destinations`) to its most recent
        end in ascending slot order, then refresh `slots` and the bitmaps."""
        torch = self.torch
        if (destinations.dim() != 2 or destinations.shape[0] != self.chains or destinations.dtype != torch.int32
                or destinations.device != self.device or destinations.stride(1) != 1):
            raise ValueError(f"destinations must be int32 [{self.chains}, count] rows on {self.device}")
        abi.check(self.library.kvip_hip_lru_commit_chains(
            ctypes.byref(self._args), self.chains, abi.ptr(destinations), destinations.stride(0),
            int(destinations.shape[1]), self.active, self._stream()), "SlotLRUChains commit")
