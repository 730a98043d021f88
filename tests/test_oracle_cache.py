"""Pins of oracle/cache.py: known answers of the reference's cache tests and brute force
against an independent model (paths relative to the KVIP reference)."""
import numpy as np

from oracle import cache as ref


def test_update_abc_known_answer():
    # tests/cache/test_abc.py:42-51
    mapping = np.full((2, 3, 2048), -1, np.int32)
    reverse = mapping.copy()
    ref.update_abc(mapping, reverse, np.array([[[1, 2, 383, 390]]], np.int32), 1, 1024, 384)
    for token in range(383, 390):
        slot = 1024 + token % 384
        assert mapping[1, 2, token] == slot
        assert reverse[1, 2, slot] == token
    assert (mapping[0] == -1).all()
    assert (reverse[1, 2, 1024:1024 + 384] >= -1).all()
    assert (reverse[1, 2, :1024] == -1).all() and (reverse[1, 2, 1408:] == -1).all()


def test_update_abc_full_ring_wrap_and_shift():
    # Descriptors of tests/cache/test_abc.py:17-31 (full 384-token ring with wrap, an empty
    # range, short ranges), shifted by 0 and 128 as that test does.
    desc = np.array([[[2, 4, 350, 734], [2, 1, 768, 768]], [[0, 3, 383, 390], [0, 2, 128, 140]]], np.int32)
    t2s = np.full((3, 5, 2048), 99, np.int32)
    s2t = t2s.copy()
    for shift in (0, 128):
        desc[:, :, 2:] += shift
        ref.update_abc(t2s, s2t, desc, 2, 1024, 384)
        begin, end = 350 + shift, 734 + shift
        ring = s2t[2, 4, 1024:1408]
        for s in range(384):
            t = next(t for t in range(begin, end) if t % 384 == s)  # exactly one token per slot
            assert ring[s] == t
        assert (s2t[2, 1, 1024:1408] == -1).all()  # empty range still clears its ring
        assert (t2s[2, 1] == 99).all()
    assert t2s[1].max() == 99 and s2t[1].max() == 99  # untouched layer


def test_update_abc_long_range_keeps_last_occupant():
    t2s = np.zeros((1, 1, 4096), np.int32)
    s2t = np.zeros((1, 1, 4096), np.int32)
    ref.update_abc(t2s, s2t, np.array([[[0, 0, 10, 1000]]], np.int32), 1, 2048, 100)
    for s in range(100):
        assert s2t[0, 0, 2048 + s] == max(t for t in range(10, 1000) if t % 100 == s)


class ListModel:
    """Independent LRU model: a Python list, oldest first."""

    def __init__(self):
        self.items, self.active = [], 0

    def resize(self, committed):
        if committed < self.active or self.active == 0 < committed:
            self.items = list(range(committed))
        elif committed > self.active:
            self.items += list(range(self.active, committed))
        self.active = committed

    def commit(self, dest):
        moved = sorted({int(d) for d in dest if 0 <= d < self.active})
        self.items = [s for s in self.items if s not in set(moved)] + moved

    def victims(self):
        v = self.items[:2048]
        return v + [-1] * (2048 - len(v))


def test_slot_lru_reference_invariants():
    # tests/cache/test_lru.py:5-15
    lru = ref.SlotLRU()
    lru.resize(16384, 16384)
    assert len(np.unique(lru.slots)) == 2048
    before = lru.slots.copy()
    lru.commit(np.array([0, 1, 2, 0], np.int32))
    assert not np.isin([0, 1, 2], lru.slots).any()
    assert len(np.unique(lru.slots)) == 2048
    assert not np.array_equal(before, lru.slots)
    lru.resize(16384, 100)
    assert (lru.slots[100:] == -1).all()


def test_slot_lru_brute_force_against_list_model():
    rng = np.random.default_rng(4)
    lru, model = ref.SlotLRU(), ListModel()
    capacity = 6000
    for step in range(120):
        if step % 17 == 0:
            committed = int(rng.integers(0, capacity + 1))
            lru.resize(capacity, committed)
            model.resize(committed)
        else:
            dest = rng.integers(-5, max(model.active, 1) + 50, int(rng.integers(0, 3000))).astype(np.int32)
            lru.commit(dest)
            model.commit(dest)
        assert lru.order() == model.items
        assert lru.slots.tolist() == model.victims()
        bits = np.zeros_like(lru.bitmap)
        for s in model.victims():
            if s >= 0:
                bits[s >> 5] |= np.uint32(1) << np.uint32(s & 31)
        assert np.array_equal(bits, lru.bitmap)


def test_publish_pages_known_answer():
    """Hand-derived: owners 2, groups 2, pages 3, block 4. Row (7, 1000, 8): index 7 is
    owner 1, group 0, page 1; row (0, 50, -1): owner 0, group 0, page 0."""
    from oracle.cache import publish_pages

    addresses = np.zeros((2, 2, 3), np.int64)
    valid = np.zeros((2, 2, 3), np.uint8)
    mapping = np.arange(20, dtype=np.int32)
    fused = (np.zeros((2, 6), np.int64), np.zeros((2, 6), np.int64))  # history 6: page 1 keeps 2 positions
    publish_pages(addresses, valid, mapping, [(7, 1000, 8), (0, 50, -1)], 4, fused, (2, 1), 656)
    assert addresses.reshape(-1).tolist() == [50, 0, 0, 0, 0, 0, 0, 1000, 0, 0, 0, 0]
    assert valid.reshape(-1).tolist() == [1, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0]
    assert mapping.tolist() == list(range(8)) + [-1] * 4 + list(range(12, 20))
    assert fused[0][1].tolist() == [0, 0, 0, 0, 1000, 1000 + 1312]
    assert fused[0][0].tolist() == [50, 50 + 1312, 50 + 2624, 50 + 3936, 0, 0]
    assert not fused[1].any()
