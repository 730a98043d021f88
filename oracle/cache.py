"""CPU restatement of KVIP's cache-state operators. TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

update_abc  - python/kvip/cache/abc.py:23-33 (the CPU branch, the reference's golden)
SlotLRU     - python/kvip/cache/lru.py:14-118 with the numba kernels of
              python/kvip/cache/_lru_kernel.py:33-199, restated as plain Python over the
              same doubly linked list (numba is not importable here, so this restatement
              is pinned by the invariants of tests/cache/test_lru.py:5-15 and by brute force
              against an independent list model in tests/test_oracle_cache.py).
publish_pages - PageUpdates.submit's CPU branch (python/kvip/cache/page_updates.py:43-62,
              the reference's golden for _page_updates_kernel.py:8-37); pinned by a hand
              known answer and the untouched-entries invariant in tests/test_oracle_cache.py.
"""
from __future__ import annotations

import numpy as np

TOPK = 2048
BITMAP_WORD_BITS = 32
BITMAP_ALIGNMENT_WORDS = 8


def update_abc(token_to_slot, slot_to_token, descriptors, requests, history, tail):
    """In place on numpy int32 arrays [layers, pool, tokens]; descriptors [groups, rows, 4]
    of (layer, owner, begin, end). For every group, for the first `requests` rows, in order:
    token_to_slot[layer, owner, begin:end] = history + t % tail, then the ring
    slot_to_token[layer, owner, history:history+tail] is reset to -1 and every token t of the
    range is written at t % tail, later tokens overwriting earlier ones (abc.py:23-33)."""
    for group in range(descriptors.shape[0]):
        for row in range(requests):
            layer, owner, begin, end = (int(v) for v in descriptors[group, row])
            for t in range(begin, end):
                token_to_slot[layer, owner, t] = history + t % tail
            ring = slot_to_token[layer, owner, history:history + tail]
            ring[:] = -1
            for t in range(begin, end):
                ring[t % tail] = t


class SlotLRU:
    """One request/layer chain; only the committed slot prefix [0, active) is evictable.

    State as in lru.py:21-31: `next`/`previous` links, `head`/`tail`, `slots` = the
    min(2048, active) oldest slots from the head (victim candidates, -1 padded) and a
    victim bitmap whose word count is rounded up to a multiple of 8."""

    def __init__(self):
        self.active = 0
        self.next = np.empty(0, np.int64)
        self.previous = np.empty(0, np.int64)
        self.head = -1
        self.tail = -1
        self.slots = np.full(TOPK, -1, np.int32)
        self.bitmap = np.zeros(0, np.uint32)
        self.version = 0

    def _words(self, capacity):
        words = (capacity + BITMAP_WORD_BITS - 1) // BITMAP_WORD_BITS
        return (words + BITMAP_ALIGNMENT_WORDS - 1) // BITMAP_ALIGNMENT_WORDS * BITMAP_ALIGNMENT_WORDS

    def _write_oldest_victims(self):
        """_lru_kernel.py:33-53: clear the bitmap, walk min(2048, active) links from head."""
        self.bitmap[:] = 0
        self.slots[:] = -1
        slot = self.head
        for index in range(min(TOPK, self.active)):
            self.slots[index] = slot
            self.bitmap[slot >> 5] |= np.uint32(1) << np.uint32(slot & 31)
            slot = int(self.next[slot])

    def _reset(self, committed):
        """_lru_kernel.py:56-99: ascending-slot-id chain over [0, committed)."""
        self.next[:] = -1
        self.previous[:] = -1
        for slot in range(committed):
            self.previous[slot] = slot - 1
            self.next[slot] = slot + 1 if slot + 1 < committed else -1
        self.head = 0
        self.tail = committed - 1

    def resize(self, capacity, committed):
        """lru.py:33-83."""
        if not 0 <= committed <= capacity:
            raise ValueError(f"cannot commit {committed} slots into a capacity of {capacity}")
        changed = False
        if capacity > len(self.next):
            capacity = max(capacity, 2 * len(self.next))
            grow = capacity - len(self.next)
            self.next = np.concatenate((self.next, np.full(grow, -1, np.int64)))
            self.previous = np.concatenate((self.previous, np.full(grow, -1, np.int64)))
            self.bitmap = np.zeros(self._words(capacity), np.uint32)
            changed = True
        if committed < self.active or self.active == 0 < committed:
            self.active = committed
            self._reset(committed)
            self._write_oldest_victims()
            self.version += 1
            return
        if committed > self.active:
            first = self.active
            for slot in range(first, committed):
                self.previous[slot] = slot - 1
                self.next[slot] = slot + 1
            self.previous[first] = self.tail
            self.next[self.tail] = first
            self.next[committed - 1] = -1
            self.tail = committed - 1
            self.active = committed
            changed = True
        if changed:
            self.version += 1
            self._write_oldest_victims()

    def commit(self, destinations):
        """lru.py:96-118 + _commit_lru_rows (_lru_kernel.py:115-199): the unique
        destinations below `active` move to the tail in ascending slot-id order. Negative
        destinations are caller errors in the reference (its caller validates, lru.py:107);
        they are ignored here, as in the device kernel."""
        dest = np.asarray(destinations, np.int64)
        dest = dest[(dest >= 0) & (dest < self.active)]
        if dest.size == 0:
            return
        for slot in sorted(set(int(s) for s in dest)):
            if slot == self.tail:
                continue
            prev, nxt = int(self.previous[slot]), int(self.next[slot])
            if prev >= 0:
                self.next[prev] = nxt
            else:
                self.head = nxt
            if nxt >= 0:
                self.previous[nxt] = prev
            self.next[self.tail] = slot
            self.previous[slot] = self.tail
            self.next[slot] = -1
            self.tail = slot
        self._write_oldest_victims()
        self.version += 1

    def order(self):
        """Slots from the head (oldest) to the tail."""
        out, slot = [], (self.head if self.active else -1)
        while slot >= 0 and len(out) <= self.active:
            out.append(slot)
            slot = int(self.next[slot])
        return out


def publish_pages(addresses, valid, token_to_slot, rows, block_size, fused=(), widths=(), token_bytes=656):
    """PageUpdates.submit (python/kvip/cache/page_updates.py:43-62), in place: addresses /
    valid [owners, groups, pages], token_to_slot flat, fused per group [owners, history]."""
    owners, groups, pages = addresses.shape
    flat_a, flat_v, flat_m = addresses.reshape(-1), valid.reshape(-1), token_to_slot.reshape(-1)
    for index, address, clear in rows:
        owner, rem = divmod(int(index), groups * pages)
        group, page = divmod(rem, pages)
        flat_a[index] = address
        flat_v[index] = 1
        if clear >= 0:
            flat_m[clear:clear + block_size] = -1
        if fused:
            table = fused[group]
            for i in range(block_size):
                pos = page * block_size + i
                if pos < table.shape[1]:
                    table[owner, pos] = address + i * widths[group] * token_bytes
