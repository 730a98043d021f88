"""GPU parity of the resident-cache LIFetch round (kvip_hip_resident_round /
kvip_hip_resident_forward) against oracle/resident.py, through the C ABI.

Bars: every output and every table the round touches is bit-exact against the oracle
(slot and logical outputs, miss counts, change records, reserved_hot, hot_valid, the
permuted Index keys / scales / addresses / logical ids, the hot KV cache), over several
consecutive rounds so that each round starts from the state the previous one left; the
reference's stateful known answer (reads 2048, 0, 4096, 2048) through the full forward
with LI and TopK on the device; errors reported in status, the failed owner's residency
cleared as the reference's CompleteEarlyUpdate does."""
import ctypes

import numpy as np
import pytest

import kvip_amd
from kvip_amd.runtime import abi
from oracle import cache as lru_ref
from oracle import indexer as li_ref
from oracle import resident as ref

pytestmark = pytest.mark.gpu
TOPK = 2048
ROW = 656


def say(*args):
    print(*args, flush=True)


class Setup:
    """Owners' Index storage with identity KV rows in a pinned host pool, the hot cache
    holding positions 0..resident-1, and a resident-mode LIFetch binding."""

    def __init__(self, torch, *, batch, owners, history, resident, q_rows, seed, heads=64, invalid=0.0,
                 row_owners=None, ring=0, prefetch=None):
        rng = np.random.default_rng(seed)
        self.torch, self.rng = torch, rng
        self.batch, self.owners, self.history, self.resident, self.q = batch, owners, history, resident, q_rows
        dev = "cuda"
        keys = rng.integers(0, 256, (owners, history, 128), dtype=np.uint8)
        keys &= 0x77  # finite fp8 e4m3 values
        self.h_keys = keys
        self.h_scales = rng.uniform(0.5, 2.0, (owners, history)).astype(np.float32)
        tokens = np.arange(owners * history).reshape(owners, history)
        self.h_addresses = (tokens * ROW).astype(np.int64)
        self.h_logical = np.broadcast_to(np.arange(history), (owners, history)).astype(np.int64).copy()
        pool = li_ref.identity_rows(tokens.reshape(-1), ROW)
        self.h_pool = pool.reshape(-1)
        self.ring = ring  # ABC ring slots after the hot ones (tail bounds bound when > 0)
        self.h_hot = np.zeros((owners, resident + ring, ROW), np.uint8)
        for o in range(owners):
            self.h_hot[o, :resident] = pool[o * history:o * history + resident]
        self.h_valid = (rng.random((owners, resident)) >= invalid).astype(np.int32)
        owners_of = np.arange(batch) if row_owners is None else np.asarray(row_owners)
        self.h_owners = owners_of.astype(np.int32)
        t = torch
        self.keys = t.from_numpy(keys).to(dev).view(t.float8_e4m3fn)
        self.scales = t.from_numpy(self.h_scales).to(dev)
        self.addresses = t.from_numpy(self.h_addresses).to(dev)
        self.logical = t.from_numpy(self.h_logical).to(dev)
        self.pool = t.empty(self.h_pool.size, dtype=t.uint8, pin_memory=True)
        self.pool.copy_(t.from_numpy(self.h_pool))
        self.hot = t.from_numpy(self.h_hot).to(dev)
        self.valid = t.from_numpy(self.h_valid).to(dev)
        self.row_owners = t.from_numpy(self.h_owners).to(dev)
        self.h_tail = np.zeros((batch, 2), np.int32)
        self.tail = t.zeros((batch, 2), dtype=t.int32, device=dev) if ring else None
        self.rot = kvip_amd.LIFetchBinding(t, batch=batch, max_context=history, device=dev, heads=heads,
                                           rows_per_request=q_rows, qk_dtype="fp8", query_ends=True)
        self.rot.seq_lens.fill_(history)
        self.rot.query_ends.fill_(history)
        self.upd = kvip_amd.ResidentIndexUpdate(
            t, keys=self.keys, scales=self.scales, addresses=self.addresses, logical_ids=self.logical,
            row_owners=self.row_owners, rotating=self.rot, hot_valid=self.valid, hot_cache=self.hot,
            host_pool=self.pool, resident=resident, tail_bounds=self.tail, prefetch=prefetch)
        self.lib = abi.load_library()

    def run_round(self, selected, lru, overlap=False):
        """Device round on the given TopK rows [batch*q, 2048] and candidates [batch, 2048]:
        kvip_hip_resident_round on one stream, or with overlap ResidentIndexUpdate.round()
        (the Fetch beside the Index update on a second stream)."""
        t = self.torch
        self.rot.topk.copy_(t.from_numpy(selected.astype(np.int32)))
        if self.tail is not None:
            self.tail.copy_(t.from_numpy(self.h_tail))
        self.upd.set_candidates(t.from_numpy(lru.astype(np.int32)).to("cuda"))
        if overlap:
            self.upd.round()
        else:
            rc = self.lib.kvip_hip_resident_round(ctypes.byref(self.upd.args), abi.stream_handle(t, self.rot.device))
            abi.check(rc, "resident round")
        t.cuda.synchronize()

    def oracle_round(self, selected, lru, prefetched=None):
        """Oracle on the host copies, request by request (each owner once per round);
        prefetched: per request, the oracle's prefetch list of the round."""
        outs = []
        for b in range(self.batch):
            o = int(self.h_owners[b])
            sel = selected[b * self.q:(b + 1) * self.q]
            reserved = ref.reserved_from_candidates(lru[b], self.resident)
            keys = self.h_keys[o].copy()
            tail = (int(self.h_tail[b, 0]), int(self.h_tail[b, 1]), self.ring) if self.ring else None
            lout, sout, res, err = ref.resident_round(
                sel, self.history, self.resident, keys, self.h_scales[o], self.h_addresses[o], self.h_logical[o],
                self.h_valid[o], reserved, lru[b], self.h_hot[o], self.h_pool, tail=tail,
                prefetched=None if prefetched is None else prefetched[b])
            self.h_keys[o] = keys
            outs.append((lout, sout, res, err, reserved))
        return outs

    def compare(self, outs):
        t = self.torch
        lo = self.upd.logical_output.cpu().numpy().reshape(self.batch, self.q, TOPK)
        so = self.upd.slot_output.cpu().numpy().reshape(self.batch, self.q, TOPK)
        counts = self.upd.miss_counts.cpu().numpy()
        status = self.upd.status.cpu().numpy()
        changes = self.upd.changes.cpu().numpy()
        cslots = self.upd.change_slots.cpu().numpy()
        reserved = self.upd.reserved_hot.cpu().numpy()
        for b, (lout, sout, res, err, rsv) in enumerate(outs):
            assert status[b] == err, (b, status[b], err)
            assert np.array_equal(reserved[b], rsv), b
            assert np.array_equal(lo[b], lout), b
            assert np.array_equal(so[b], sout), b
            if err:
                continue
            added = list(res["added"]) + [0] * (4 - len(res["added"]))
            assert counts[b].tolist() == added + [int(res["added"].sum())], b
            assert np.array_equal(changes[b], res["changes"]), b
            assert np.array_equal(cslots[b], res["change_slots"]), b
        assert np.array_equal(self.keys.view(t.uint8).cpu().numpy(), self.h_keys)
        assert np.array_equal(self.scales.cpu().numpy(), self.h_scales)
        assert np.array_equal(self.addresses.cpu().numpy(), self.h_addresses)
        assert np.array_equal(self.logical.cpu().numpy(), self.h_logical)
        assert np.array_equal(self.valid.cpu().numpy(), self.h_valid)
        assert np.array_equal(self.hot.cpu().numpy(), self.h_hot)


def mtp_selection(rng, q_rows, history, resident, hot_frac, n=None, hot_pool=None):
    """Rows of one request sharing most of their selection (decode + MTP)."""
    n = int(rng.integers(1500, TOPK + 1)) if n is None else n
    hot_src = np.arange(resident) if hot_pool is None else hot_pool
    hot = rng.choice(hot_src, int(n * hot_frac), replace=False)
    cold = rng.choice(np.arange(resident, history), n - len(hot), replace=False)
    base = rng.permutation(np.concatenate([hot, cold]))
    out = np.full((q_rows, TOPK), -1, np.int64)
    for q in range(q_rows):
        row = base.copy()
        swap = rng.random(n) < 0.1
        row[swap] = rng.choice(np.setdiff1d(np.arange(history), base), int(swap.sum()), replace=False)
        out[q, :n] = rng.permutation(row)
    return out


@pytest.mark.parametrize("batch,owners,q_rows,history,resident,seed,dups", [
    (2, 2, 1, 8192, 4096, 1, False),
    (3, 3, 1, 16384, 4096, 4, True),   # one row per request, with repeated tokens inside rows
    (3, 4, 4, 16384, 8192, 2, False),
    (4, 4, 2, 12288, 2048, 3, True),
])
def test_resident_round_matches_oracle_over_rounds(torch_gpu, batch, owners, q_rows, history, resident, seed, dups):
    """Consecutive rounds against the oracle. dups: 5 % of every row's entries repeat another
    entry of the same row (the first occurrence takes the miss rank, the repeats its slot)."""
    torch = torch_gpu
    say(f"case resident round b={batch} o={owners} q={q_rows} h={history} r={resident} seed={seed} dups={dups}")
    owners_of = np.random.default_rng(seed).permutation(owners)[:batch]
    st = Setup(torch, batch=batch, owners=owners, history=history, resident=resident, q_rows=q_rows, seed=seed,
               invalid=0.05, row_owners=owners_of)
    rng = st.rng
    policies = []
    for b in range(batch):
        p = lru_ref.SlotLRU()
        p.resize(resident, resident)
        policies.append(p)
    for rnd in range(3):
        say(f"  round {rnd}")
        selected = np.concatenate([mtp_selection(rng, q_rows, history, resident, 0.6) for _ in range(batch)])
        if dups:
            for row in selected:
                n = int((row >= 0).sum())
                at = rng.choice(n, n // 20, replace=False)
                row[at] = row[rng.integers(0, n, len(at))]
        lru = np.stack([p.slots.astype(np.int64) for p in policies])
        outs = st.oracle_round(selected, lru)
        st.run_round(selected, lru)
        st.compare(outs)
        for b, p in enumerate(policies):
            s = outs[b][1]
            p.commit(s[s >= 0])


def test_resident_round_abc_tail_matches_oracle(torch_gpu):
    """ABC tail bounds over three rounds (the tail grows by a decode step each round): a
    tail longer than the ring (its last positions are ordinary misses), a tail inside the
    hot range (hot, valid positions that must not count as hits) and an empty tail; every
    row also selects ~15 % tail positions. Everything bit-exact against the oracle."""
    torch = torch_gpu
    batch, q_rows, history, resident, ring = 3, 4, 16384, 4096, 512
    say(f"case resident abc tail b={batch} q={q_rows} h={history} r={resident} ring={ring}")
    st = Setup(torch, batch=batch, owners=batch, history=history, resident=resident, q_rows=q_rows, seed=11,
               invalid=0.05, ring=ring)
    rng = st.rng
    policies = []
    for _ in range(batch):
        p = lru_ref.SlotLRU()
        p.resize(resident, resident)
        policies.append(p)
    tails = np.array([[15000, 15600], [1000, 1300], [0, 0]], np.int32)
    for rnd in range(3):
        say(f"  round {rnd}")
        st.h_tail = tails + np.array([[0, 2], [0, 2], [0, 0]], np.int32) * rnd
        rows = []
        for b in range(batch):
            sel = mtp_selection(rng, q_rows, history, resident, 0.6, n=2048)
            lo, hi = map(int, st.h_tail[b])
            if hi > lo:
                picks = rng.choice(np.arange(lo, hi), min(300, hi - lo), replace=False)
                for q in range(q_rows):
                    row = sel[q]
                    keep = ~np.isin(row, picks)
                    row = np.concatenate([row[keep], picks])[:TOPK]
                    row = row[np.unique(row, return_index=True)[1]]
                    pad = np.setdiff1d(np.arange(resident, history), row)[:TOPK - len(row)]
                    sel[q] = rng.permutation(np.concatenate([row, pad]))
            rows.append(sel)
        selected = np.concatenate(rows)
        lru = np.stack([p.slots.astype(np.int64) for p in policies])
        outs = st.oracle_round(selected, lru)
        for b, (lout, sout, res, err, rsv) in enumerate(outs):
            assert err == 0, (b, err)
            lo, hi = map(int, st.h_tail[b])
            sel = selected[b * q_rows:(b + 1) * q_rows]
            mapped = (sel >= lo) & (sel < min(hi, lo + ring))
            assert np.array_equal(sout[mapped], resident + sel[mapped] % ring), b
            beyond = sel[(sel >= lo + ring) & (sel < hi)]
            assert np.isin(beyond, res["tokens"]).all(), b  # unmapped tail positions are misses
        st.run_round(selected, lru)
        st.compare(outs)
        for b, p in enumerate(policies):
            s = outs[b][1]
            p.commit(s[(s >= 0) & (s < resident)])


def test_resident_forward_stateful_known_answer(torch_gpu):
    """correctness.py:170-228 through the whole forward on the device (LI, TopK, round),
    the device SlotLRU supplying candidates: reads 2048, 0, 4096, 2048 per request."""
    torch = torch_gpu
    batch, history, resident, heads = 2, 12288, 4096, 32
    st = Setup(torch, batch=batch, owners=batch, history=history, resident=resident, q_rows=4, seed=7, heads=heads)
    keys = np.zeros((batch, history, 128), np.uint8)
    for feature, begin in enumerate((4096, 6144, 8192)):
        keys[:, begin:begin + 2048, feature] = 0x38  # exactly 1 in e4m3
    st.keys.view(torch.uint8).copy_(torch.from_numpy(keys))
    st.valid.fill_(1)
    rot, upd = st.rot, st.upd
    rot.weights.fill_(1.0)
    rot.query_ends.copy_(torch.arange(history - 3, history + 1, dtype=torch.int32).repeat(batch))
    fwd = kvip_amd.LIFetch(rot, upd)
    lrus = [kvip_amd.SlotLRU("cuda") for _ in range(batch)]
    for p in lrus:
        p.resize(resident, resident)
    reads = []
    for number in range(1, 5):
        features = (1, 2, 1, 2) if number == 3 else (0, 0, 0, 0)
        query = torch.zeros((batch, 4, heads, 128), dtype=torch.float32)
        for q, feature in enumerate(features):
            query[:, q, :, feature] = 1.0
        rot.query.copy_(query.view(batch * 4, heads, 128).to(torch.float8_e4m3fn))
        upd.set_candidates(torch.cat([p.slots for p in lrus]))
        say(f"  stateful round {number}")
        fwd()
        torch.cuda.synchronize()
        assert not upd.status.any(), upd.status.cpu().tolist()
        counts = upd.miss_counts.cpu().numpy()
        reads.append(counts[:, 4].tolist())
        slots = upd.slot_output.view(batch, -1)
        for b, p in enumerate(lrus):
            p.commit(slots[b][slots[b] >= 0].contiguous())
        logical = st.logical.cpu().numpy()
        valid = st.valid.cpu().numpy()
        expected = set(range(6144, 10240)) if number == 3 else set(range(4096, 6144))
        for b in range(batch):
            hot = set(logical[b, :resident][valid[b] != 0].tolist())
            assert expected <= hot, (number, b)
            if number == 3:
                assert not hot & set(range(4096, 6144))
            # Every selected slot holds its token's KV (identity rows of owner b).
            lo = upd.logical_output.view(batch, -1)[b].cpu().numpy()
            so = slots[b].cpu().numpy()
            pool = st.h_pool.reshape(-1, ROW)
            hotc = st.hot[b].cpu().numpy()
            assert np.array_equal(hotc[so], pool[b * history + lo])
    assert reads == [[2048, 2048], [0, 0], [4096, 4096], [2048, 2048]]


@pytest.mark.parametrize("overlap", [False, True], ids=["one_stream", "fetch_beside_update"])
def test_resident_errors_clear_the_owner_residency(torch_gpu, overlap):
    """Failure contract of the reference (index_cache_update.h:5-21): a failed request's
    owner loses all residency; a request failing before the Fetch publishes -1 and moves
    nothing. Checked against the oracle on every table, then over a second round in which
    that owner reads every position cold; the same with the Fetch beside the Index update."""
    torch = torch_gpu
    st = Setup(torch, batch=2, owners=2, history=8192, resident=4096, q_rows=1, seed=9)
    run = st.run_round
    st.run_round = lambda sel, lru: run(sel, lru, overlap=overlap)
    rng = st.rng
    selected = np.concatenate([mtp_selection(rng, 1, 8192, 4096, 0.5) for _ in range(2)])
    lru = np.stack([np.arange(2048), np.arange(2048, 4096)])
    lru[1, 5] = 9999  # outside the hot range: request 1 fails, request 0 runs
    say("case candidate outside the hot range")
    st.run_round(selected, lru)
    outs = st.oracle_round(selected, lru)
    st.compare(outs)
    status = st.upd.status.cpu().numpy()
    assert status[0] == 0 and status[1] & abi.RESIDENT_ERR_CANDIDATE
    assert (st.upd.slot_output[1].cpu() == -1).all() and (st.upd.logical_output[1].cpu() == -1).all()
    assert not st.valid[1].any() and st.valid[0].any()
    # Duplicate candidates (advisor case): both ordinals would get the same slot.
    say("case duplicate candidates, then a cold round")
    lru = np.stack([np.arange(2048, 4096), np.arange(2048, 4096)])
    lru[0, 17] = lru[0, 1900]
    selected = np.concatenate([mtp_selection(rng, 1, 8192, 4096, 0.6) for _ in range(2)])
    st.run_round(selected, lru)
    st.compare(st.oracle_round(selected, lru))
    status = st.upd.status.cpu().numpy()
    assert status[0] == abi.RESIDENT_ERR_CANDIDATE and status[1] == 0
    assert not st.valid[0].any()
    lru = np.stack([np.arange(2048), np.arange(2048)])
    selected = np.concatenate([mtp_selection(rng, 1, 8192, 4096, 0.6, n=1800) for _ in range(2)])
    st.run_round(selected, lru)
    outs = st.oracle_round(selected, lru)
    st.compare(outs)
    counts = st.upd.miss_counts.cpu().numpy()
    assert counts[0, 4] == 1800  # every selected position of the cleared owner is a miss
    assert not st.upd.status.any()
    # A KV address outside the host pool fails the request before anything is fetched.
    say("case source outside the host pool")
    st2 = Setup(torch, batch=1, owners=1, history=8192, resident=4096, q_rows=1, seed=10)
    run2 = st2.run_round
    st2.run_round = lambda sel, lru: run2(sel, lru, overlap=overlap)
    st2.addresses[0, 5000] = st2.pool.numel()
    st2.h_addresses[0, 5000] = st2.pool.numel()
    sel = np.full((1, TOPK), -1, np.int64)
    sel[0, :3] = [5000, 6000, 7000]
    hot_before = st2.hot.clone()
    st2.run_round(sel, np.arange(2048)[None, :])
    st2.compare(st2.oracle_round(sel, np.arange(2048)[None, :]))
    assert st2.upd.status.cpu().numpy()[0] & abi.RESIDENT_ERR_SOURCE
    assert torch.equal(st2.hot, hot_before) and not st2.valid.any()


def test_resident_round_overlap_equals_sequential(torch_gpu):
    """ResidentIndexUpdate.round() with the Fetch beside the Index update and the attached
    LRU commit (two streams) leaves exactly the state of kvip_hip_resident_round followed by
    the commit on one stream: every table, output, hot-cache row and LRU chain, over
    consecutive rounds whose victim candidates come from the chains, first eagerly, then
    replayed from one captured graph (with eager work between replays); one request fails
    in round 3 (a candidate outside the hot range)."""
    torch = torch_gpu
    batch, history, resident = 3, 8192, 4096
    a = Setup(torch, batch=batch, owners=batch, history=history, resident=resident, q_rows=2, seed=21)
    b = Setup(torch, batch=batch, owners=batch, history=history, resident=resident, q_rows=2, seed=21)
    chains_a = kvip_amd.SlotLRUChains(torch, batch, resident, "cuda", slots=a.upd.lru_slots)
    chains_b = kvip_amd.SlotLRUChains(torch, batch, resident, "cuda", slots=b.upd.lru_slots)
    a.upd.attach_lru(chains_a)
    rows_b = b.upd.slot_output.view(batch, -1)
    stream = abi.stream_handle(torch, "cuda")

    def tables(st, chains):
        u = st.upd
        return [st.keys.view(torch.uint8), st.scales, st.addresses, st.logical, st.valid, st.hot, u.outputs,
                u.miss_counts, u.status, u.changes, u.change_slots, u.reserved_hot, u.lru_slots, chains.order,
                chains.bitmap]

    rng = np.random.default_rng(4)
    graph = None
    for step in range(6):
        sel = np.concatenate([mtp_selection(rng, 2, history, resident, 0.7) for _ in range(batch)])
        say(f"round {step} ({'eager' if step < 2 else 'graph replay'})")
        for st in (a, b):
            st.rot.topk.copy_(torch.from_numpy(sel.astype(np.int32)))
            if step == 3:
                st.upd.lru_slots[1, 7] = resident + 5
        if step < 2:
            a.upd.round()
        else:
            if graph is None:
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    a.upd.round()
            graph.replay()
        abi.check(b.lib.kvip_hip_resident_round(ctypes.byref(b.upd.args), stream), "resident round")
        chains_b.commit(rows_b)
        torch.cuda.synchronize()
        for x, y in zip(tables(a, chains_a), tables(b, chains_b)):
            assert torch.equal(x, y), step
        status = a.upd.status.cpu().numpy()
        if step == 3:
            assert status[1] & abi.RESIDENT_ERR_CANDIDATE and not a.valid[1].any()
        else:
            assert not status.any(), (step, status)
        assert int(a.upd.miss_counts[:, 4].sum()) > 0


def oracle_prefetch(st, keys, lru, pf):
    """The oracle's prefix classification and prefetch of every request on the device keys."""
    out = []
    cold_len = st.history - st.resident
    cold_words = (st.rot.key_stride - st.resident + 31) // 32
    for b in range(st.batch):
        victim = np.zeros((st.q, TOPK), bool)
        cold = np.zeros((st.q, cold_len), bool)
        for q in range(st.q):
            r = b * st.q + q
            _, _, vbits, cbits = ref.prefix_classify(keys[r], st.history, st.resident, lru[b], cold_words)
            victim[q] = np.unpackbits(vbits.view(np.uint8), bitorder="little").astype(bool)
            cold[q] = np.unpackbits(cbits.view(np.uint8), bitorder="little")[:cold_len].astype(bool)
        tail = (int(st.h_tail[b, 0]), int(st.h_tail[b, 1]), st.ring) if st.ring else None
        out.append(ref.prefetch(victim, cold, lru[b], st.history, st.resident, tail=tail, windows=pf.windows,
                                prefetch_limit=pf.prefetch_limit, window_limit=pf.window_limit))
    return out


@pytest.mark.parametrize("q_rows,ring,windowed", [(1, 0, False), (1, 0, True), (2, 512, False)])
def test_resident_prefetch_forward_matches_oracle(torch_gpu, q_rows, ring, windowed):
    """The forward with the speculative windowed prefetch (prefix TopK and hit bits, the
    window scan and budgets, the prefetch Fetch on a second stream, the final round with
    prefetched tokens resolved to their slots and the prefetch applied first in the Index
    update) over three rounds against the oracle, bit-exact: prefetch records, outputs,
    change records, Index tables, residency and the hot cache; the queries drift from round
    to round so that each round prefetches, hits and misses."""
    torch = torch_gpu
    batch, history, resident = 3, 16384, 4096
    pf = kvip_amd.ResidentPrefetch(windows=4, prefetch_limit=600, window_limit=200, windowed=windowed)
    say(f"case resident prefetch q={q_rows} ring={ring} windowed={windowed}")
    st = Setup(torch, batch=batch, owners=batch, history=history, resident=resident, q_rows=q_rows, seed=13 + ring,
               invalid=0.03, ring=ring, prefetch=pf)
    rot, upd = st.rot, st.upd
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    base = torch.randn(rot.query.shape, generator=gen, device="cuda")
    rot.weights.copy_(torch.randn(rot.weights.shape, generator=gen, device="cuda").abs() / 8)
    if ring:
        st.h_tail = np.array([[history - 300, history], [2000, 2600], [0, 0]], np.int32)
    policies = []
    for _ in range(batch):
        p = lru_ref.SlotLRU()
        p.resize(resident, resident)
        policies.append(p)
    fwd = kvip_amd.LIFetch(rot, upd)
    assert fwd.windowed == windowed
    for rnd in range(3):
        say(f"  round {rnd}")
        q = base + 0.4 * rnd * torch.randn(base.shape, generator=gen, device="cuda")
        rot.query.copy_(q.clamp(-8, 8).to(torch.float8_e4m3fn))
        lru = np.stack([p.slots.astype(np.int64) for p in policies])
        upd.set_candidates(torch.from_numpy(lru.astype(np.int32)).cuda())
        if st.tail is not None:
            st.tail.copy_(torch.from_numpy(st.h_tail))
        fwd()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        keys = rot.score_keys.cpu().numpy().view(np.uint16)
        top = rot.topk.cpu().numpy().astype(np.int64)
        for r in range(batch * q_rows):
            assert np.array_equal(top[r], li_ref.topk_reference(keys[r], history)), r
        pre = oracle_prefetch(st, keys, lru, pf)
        counts = upd.prefetch_counts.cpu().numpy()
        tokens = upd.prefetch_tokens.cpu().numpy()
        for b in range(batch):
            assert counts[b] == len(pre[b]), (b, counts[b], len(pre[b]))
            assert tokens[b, :counts[b]].tolist() == [t for t, _ in pre[b]], b
        say(f"    prefetched {counts.tolist()}, final misses {upd.miss_counts[:, 4].cpu().tolist()}")
        assert counts.sum() > 0
        outs = st.oracle_round(top, lru, prefetched=pre)
        st.compare(outs)
        for b, p in enumerate(policies):
            s_out = outs[b][1]
            p.commit(s_out[(s_out >= 0) & (s_out < resident)])


@pytest.mark.parametrize("prefetch,q_rows,windowed", [(False, 2, False), (True, 2, False), (True, 1, True)])
def test_resident_forward_graph_replay(torch_gpu, prefetch, q_rows, windowed):
    """The resident forward captured once and replayed: each replay equals the same step
    run eagerly on a copy of the state (tables and outputs); with the prefetch, the capture
    forks the prefetch onto its second stream and joins it before the final round (one
    query row: the windowed prefetch, scoring window by window with the decisions on a
    second stream and the host copies on a third)."""
    torch = torch_gpu
    say(f"case resident graph replay prefetch={prefetch} q={q_rows} windowed={windowed}")
    st = Setup(torch, batch=2, owners=2, history=8192, resident=4096, q_rows=q_rows, seed=12,
               prefetch=kvip_amd.ResidentPrefetch(windows=3, prefetch_limit=300, windowed=windowed)
               if prefetch else None)
    rot, upd = st.rot, st.upd
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    rot.query.copy_(torch.randn(rot.query.shape, generator=gen, device="cuda").clamp(-8, 8).to(torch.float8_e4m3fn))
    rot.weights.copy_(torch.randn(rot.weights.shape, generator=gen, device="cuda") / 8)
    upd.set_candidates(torch.stack([torch.arange(2048), torch.arange(2048, 4096)]).int().cuda())
    fwd = kvip_amd.LIFetch(rot, upd)
    assert not prefetch or fwd.windowed == windowed
    state = (st.keys, st.scales, st.addresses, st.logical, st.valid, st.hot)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fwd()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    for step in range(3):
        start = [x.clone() for x in state]
        graph.replay()
        torch.cuda.synchronize()
        got = [x.clone() for x in state] + [upd.outputs.clone(), upd.miss_counts.clone()]
        if prefetch:
            got.append(upd.prefetch_counts.clone())
        for x, s in zip(state, start):
            x.copy_(s)
        upd.outputs.fill_(-9)
        fwd()
        torch.cuda.synchronize()
        want = [x for x in state] + [upd.outputs, upd.miss_counts]
        if prefetch:
            want.append(upd.prefetch_counts)
        for g, w in zip(got, want):
            assert torch.equal(g, w), step
        assert not upd.status.any()


@pytest.mark.parametrize("ctx,ends,resident", [
    ([20000, 9000], [20000, 19990, 9000, 1500], 4096),
    # Rows longer than the register select's 65536 keys, prefix of 16384 (config 4's shape).
    ([70000, 40000], [70000, 69000, 40000, 16000], 16384),
])
def test_resident_prefix_matches_oracle(torch_gpu, ctx, ends, resident):
    """Resident TopK, threshold and hit bits on the device keys of a scored step equal the
    oracle's on the same keys (bit-exact), including short and query-bounded rows."""
    torch = torch_gpu
    from kvip_amd import synthetic

    wl = synthetic.decode_workload(torch, batch=2, ctx=ctx, device="cuda", seed=21, rows_per_request=2)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl, query_ends=ends)
    fwd.score()
    rng = np.random.default_rng(21)
    lru = np.stack([rng.permutation(resident)[:2048] for _ in range(2)]).astype(np.int32)
    lru[0, :2] = [resident + 3, -1]
    pre = kvip_amd.ResidentPrefix(torch, rot, torch.from_numpy(lru).cuda(), resident)
    say(f"case resident prefix ctx {ctx} resident {resident}")
    pre()
    torch.cuda.synchronize()
    keys = rot.score_keys.cpu().numpy().view(np.uint16)
    for r in range(rot.rows):
        valid = min(int(wl.ctx[r // 2]), ends[r])
        sel, thr, victim, cold = ref.prefix_classify(keys[r], valid, resident, lru[r // 2], pre.cold_words)
        assert np.array_equal(pre.prefix_topk[r].cpu().numpy(), sel), r
        assert int(pre.thresholds[r].item()) & 0xFFFF == thr, r
        assert np.array_equal(pre.victim_hits[r].cpu().numpy().view(np.uint32), victim), r
        assert np.array_equal(pre.cold_hits[r, :pre.cold_words].cpu().numpy().view(np.uint32), cold), r
