"""GPU parity of the vLLM indexer selector (kvip_amd.VllmIndexSelector over QueryInputs,
IndexCacheStorage, the resident LIFetch forward and PagedIndexer) against the oracle,
through the C ABI, over three consecutive scheduler steps sharing one Index storage:

  A  prefill only: restored prefixes and new tokens imported into the Index storage, and
     native selection of every prefill row (four sequences in one call);
  B  decode only (one to four MTP tokens per request, one empty request row): decode
     ingest, query packing, LI, TopK, the resident round, outputs in token order;
  C  mixed: decode requests through the forward, prefill requests (a new owner with a
     restored prefix, a continuing chunk) through native selection, assembled in token
     order.

Bars: Index storage (keys, scales, addresses, logical ids, hot validity) and the hot KV
cache bit-exact against the oracle after every step; LI scores within 3e-2 and keys
bit-identical on more than 97% of each row's significant keys, TopK bit-exact on the device keys and inside the oracle's
one-ulp cutoff band; logical and slot outputs bit-exact against the oracle's resident
round on the device TopK, published in token order (oracle.adapters.publish_outputs)."""
from types import SimpleNamespace

import numpy as np
import pytest

import kvip_amd
from oracle import adapters as ad
from oracle import indexer as li
from oracle import resident as rs

pytestmark = pytest.mark.gpu
TOPK = 2048
ROW = 656
B, OWNERS, HISTORY, RESIDENT, HEADS = 4, 6, 8192, 4096, 64
MAXB = HISTORY // 128


def say(*args):
    print(*args, flush=True)


class World:
    """Paged vLLM index cache (each request owns 64 private pages), the Index storage of six
    owners, a pinned host KV pool of identity rows, the hot cache and the selector."""

    def __init__(self, torch, seed, ring=0):
        self.torch, self.rng = torch, np.random.default_rng(seed)
        self.ring = ring  # ABC ring slots after the hot ones (the update then binds tail bounds)
        self.h_tail = np.zeros((B, 2), np.int32)
        rng, t, dev = self.rng, torch, "cuda"
        blocks = 5 * MAXB + 8
        self.h_cache_keys = rng.integers(0, 256, (blocks, 128, 128), dtype=np.uint8) & 0x77
        self.h_cache_scales = rng.uniform(0.5, 2.0, (blocks, 128)).astype(np.float32)
        self.cache_keys = t.from_numpy(self.h_cache_keys).to(dev).view(t.float8_e4m3fn)
        self.cache_scales = t.from_numpy(self.h_cache_scales).to(dev)
        perm = rng.permutation(blocks)
        self.pages = {o: perm[(o - 1) * MAXB:o * MAXB].astype(np.int32) for o in range(1, OWNERS)}
        pool = li.identity_rows(np.arange(OWNERS * HISTORY), ROW)
        self.h_pool = pool.reshape(-1)
        self.pool = t.empty(self.h_pool.size, dtype=t.uint8, pin_memory=True)
        self.pool.copy_(t.from_numpy(self.h_pool))
        self.storage = kvip_amd.IndexCacheStorage(t, OWNERS, HISTORY, RESIDENT, dev)
        self.hot = t.zeros((OWNERS, RESIDENT + ring, ROW), dtype=t.uint8, device=dev)
        self.tail = t.zeros((B, 2), dtype=t.int32, device=dev) if ring else None
        self.inputs = kvip_amd.QueryInputs(t, B, dev, history=HISTORY)
        self.rot = kvip_amd.LIFetchBinding(t, batch=B, max_context=HISTORY, device=dev, heads=HEADS, rows_per_request=4,
                                           qk_dtype="fp8", weight_dtype=t.bfloat16,
                                           query_ends=True).bind_query_inputs(self.inputs)
        s = self.storage
        self.update = kvip_amd.ResidentIndexUpdate(
            t, keys=s.keys.view(t.float8_e4m3fn), scales=s.scales, addresses=s.addresses, logical_ids=s.logical_ids,
            row_owners=self.inputs.row_owners, rotating=self.rot, hot_valid=s.hot_valid, hot_cache=self.hot,
            host_pool=self.pool, resident=RESIDENT, query_inputs=self.inputs, tail_bounds=self.tail)
        self.indexer = kvip_amd.PagedIndexer(t, keys=self.cache_keys, scales=self.cache_scales, max_rows=128,
                                             max_context=HISTORY, device=dev, heads=HEADS, max_sequences=4)
        self.selector = kvip_amd.VllmIndexSelector(t, inputs=self.inputs, rotating=self.rot, update=self.update,
                                                   logical_ids=s.logical_ids, row_owners=self.inputs.row_owners,
                                                   storage=s)
        self.imported = set()  # the oracle's record of owners whose prefix was imported

    def snapshot(self):
        s, t = self.storage, self.torch
        return dict(keys=s.keys.cpu().numpy(), scales=s.scales.cpu().numpy(), addresses=s.addresses.cpu().numpy(),
                    logical=s.logical_ids.cpu().numpy(), valid=s.hot_valid.cpu().numpy(), hot=self.hot.cpu().numpy())

    def step(self, requests):
        """requests: (owner, request id, start, count, decode). Returns the step's device
        result, the oracle's state after the step and the host inputs."""
        t, rng = self.torch, self.rng
        plans, positions, slots, begin = [], [], [], 0
        for owner, request, start, count, decode in requests:
            pos = np.arange(start, start + count)
            positions.append(pos)
            slots.append(self.pages[owner][pos // 128].astype(np.int64) * 128 + pos % 128)
            key_end = t.tensor([start + count], dtype=t.int32, device="cuda")
            query_end = t.tensor([count], dtype=t.int32, device="cuda")
            plans.append(kvip_amd.RequestPlan(owner=owner, request=request, begin=begin, stop=begin + count,
                                              start=start, decode=decode, query_end=query_end, key_end=key_end))
            begin += count
        tokens = begin
        positions, slots = np.concatenate(positions), np.concatenate(slots)
        table = np.stack([self.pages[r[0]] for r in requests])
        # Queries: the MTP tokens of a decode request share their query, weights and scales
        # (their selections then overlap, as consecutive draft tokens' do).
        q = np.empty((tokens, HEADS, 128), np.float32)
        w = np.empty((tokens, HEADS), np.float32)
        sc = np.empty((tokens, HEADS), np.float32)
        for p, (owner, request, start, count, decode) in zip(plans, requests):
            n = 1 if decode else count
            qq = rng.standard_normal((n, HEADS, 128)).astype(np.float32)
            ww = rng.standard_normal((n, HEADS)).astype(np.float32)
            ss = rng.uniform(0.5, 2.0, (n, HEADS)).astype(np.float32)
            q[p.begin:p.stop], w[p.begin:p.stop], sc[p.begin:p.stop] = qq, ww, ss
        query = t.from_numpy(q).to(t.float8_e4m3fn).cuda()
        weights = t.from_numpy(w).to(t.bfloat16).cuda()
        scale = t.from_numpy(sc).cuda()
        metadata = SimpleNamespace(
            slot_mapping=t.from_numpy(slots).cuda(), block_table=t.from_numpy(table).cuda(), block_size=128,
            cum_query_lens=t.tensor(np.cumsum([r[3] for r in requests]), dtype=t.int32, device="cuda"),
            seq_lens=t.tensor([r[2] + r[3] for r in requests], dtype=t.int32, device="cuda"))
        sel = self.selector
        sel.prepare(plans)
        for owner, request, start, count, decode in requests:
            pages = (start + count + 127) // 128
            base = owner * HISTORY
            self.storage.publish(owner, [(base + j * 128) * ROW for j in range(pages)], block_size=128,
                                 token_bytes=ROW)
        sel.positions = t.from_numpy(positions).cuda()
        decodes = [r for r in requests if r[4]]
        if decodes:
            self.inputs.bind_positions(sel.positions)
        lru = np.stack([rng.permutation(RESIDENT)[:TOPK] for _ in range(B)]).astype(np.int32)
        self.update.set_candidates(t.from_numpy(lru).cuda())
        state = self.snapshot()
        say(f"  step: {len(requests)} requests, {tokens} tokens, {len(decodes)} decode")
        out = sel(query, weights, self.indexer, metadata, scale)
        t.cuda.synchronize()
        host = SimpleNamespace(plans=plans, requests=requests, positions=positions, slots=slots, table=table,
                               q=li.fp8_e4m3_decode(query.view(t.uint8).cpu().numpy()),
                               w=weights.float().cpu().numpy(), s=sc, lru=lru, tokens=tokens)
        return out, state, host

    # ---- oracle -------------------------------------------------------------------
    def oracle_ingest(self, state, host, mixed_or_prefill):
        src_k = self.h_cache_keys.reshape(-1, 128)
        src_s = self.h_cache_scales.reshape(-1)
        if mixed_or_prefill:
            plans = [(p.owner, p.start, p.begin, p.stop) for p in host.plans]
            ad.ingest_prefill(state["keys"], state["scales"], src_k, src_s, host.table, 128, host.slots, plans,
                              host.positions, self.imported)
            return None, None
        dec = [r for r in host.requests if r[4]]
        meta = ad.prepare_metadata(B, [r[3] for r in dec], [p.begin for p in host.plans if p.decode],
                                   [r[0] for r in dec])
        ends = ad.bind_positions(meta, host.positions)
        owners = meta[4].view(np.int32)[:B]
        ad.ingest_decode(state["keys"], state["scales"], src_k, src_s, host.slots, meta, ends, owners, HISTORY)
        return meta, ends

    def check_prefill_rows(self, got, host, plan_rows, exact_keys=None):
        """Native selection of prefill requests (plan index, rows of `got` [n, 2048])."""
        fk = li.fp8_e4m3_decode(self.h_cache_keys)
        for i, rows in plan_rows:
            p = host.plans[i]
            count, key_end = p.stop - p.begin, p.start + p.stop - p.begin
            cu = np.array([0, count])
            want, vis = li.prefill_keys_paged(host.q[p.begin:p.stop], host.w[p.begin:p.stop], host.s[p.begin:p.stop],
                                              fk, self.h_cache_scales, host.table[i:i + 1], cu,
                                              np.array([key_end]), HISTORY)
            for j in range(count):
                v = int(vis[j])
                sel = rows[j]
                if v < TOPK:
                    assert sorted(sel[sel >= 0].tolist()) == list(range(v)), (i, j)
                else:
                    assert li.validate_topk_band(sel, li.score_values(want[j, :v])), (i, j)

    def check_decode(self, state, host, meta, ends, out_rows):
        """LI keys and TopK of the packed rows, the resident round and token-order outputs."""
        t = self.torch
        pq, pw, ps = ad.pack(meta, host.q, host.w, host.s)
        owners = meta[4].view(np.int32)[:B]
        got_keys = self.rot.score_keys.cpu().numpy().view(np.uint16)
        got_top = self.rot.topk.cpu().numpy()
        fkeys = li.fp8_e4m3_decode(state["keys"])
        want = np.zeros_like(got_keys)
        valid = ends.astype(np.int64)
        for r in range(B * 4):
            v = int(valid[r])
            if v:
                o = int(owners[r // 4])
                want[r, :v] = li.li_keys(pq[r], fkeys[o, :v], pw[r], ps[r], state["scales"][o, :v])
        # Scores within 3e-2 (relative, plus 3e-2 of the row's largest) and, per row, more
        # than 97% of the significant keys bit-identical: signed bf16 weights make the
        # 64-head sums cancel more than in the other suites, so more sums sit within the
        # device's fp32 accumulation error of a bf16 rounding boundary.
        for r in range(B * 4):
            v = int(valid[r])
            if v:
                g = li.score_values(got_keys[r, :v]).astype(np.float64)
                x = li.score_values(want[r, :v]).astype(np.float64)
                assert not (np.abs(g - x) > 3e-2 * np.abs(x) + 3e-2 * np.abs(x).max()).any(), r
                share = li.identical_share(got_keys[r:r + 1], want[r:r + 1], valid[r:r + 1])
                say(f"    row {r}: {v} keys, identical share {share:.4f}")
                assert share > 0.97, r
        for r in range(B * 4):
            v = int(valid[r])
            assert np.array_equal(got_top[r], li.topk_reference(got_keys[r], v)), r
            if v >= TOPK:
                assert li.validate_topk_band(got_top[r], li.score_values(want[r, :v])), r
        # Resident round on the device TopK, request by request.
        lout = np.full((B * 4, TOPK), -1, np.int32)
        sout = np.full((B * 4, TOPK), -1, np.int32)
        for b in range(B):
            o = int(owners[b])
            reserved = rs.reserved_from_candidates(host.lru[b], RESIDENT)
            keys = state["keys"][o].copy()
            tail = (int(self.h_tail[b, 0]), int(self.h_tail[b, 1]), self.ring) if self.ring else None
            lo, so, res, err = rs.resident_round(
                got_top[b * 4:(b + 1) * 4], HISTORY, RESIDENT, keys, state["scales"][o], state["addresses"][o],
                state["logical"][o], state["valid"][o], reserved, host.lru[b], state["hot"][o], self.h_pool,
                tail=tail)
            state["keys"][o] = keys
            assert err == 0, (b, err)
            lout[b * 4:(b + 1) * 4], sout[b * 4:(b + 1) * 4] = lo, so
        assert not self.update.status.any(), self.update.status.cpu().tolist()
        want_l, want_s = ad.publish_outputs(meta, lout), ad.publish_outputs(meta, sout)
        assert np.array_equal(self.update.logical_output[:, 0].cpu().numpy(), want_l)
        assert np.array_equal(self.update.slot_output[:, 0].cpu().numpy(), want_s)
        tokens = int(meta[3].sum())
        assert np.array_equal(out_rows, want_l[:tokens])
        assert np.array_equal(self.selector.slots(tokens)[:, 0].cpu().numpy(), want_s[:tokens])

    def check_state(self, state):
        got = self.snapshot()
        for name in ("keys", "scales", "addresses", "logical", "valid", "hot"):
            assert np.array_equal(got[name], state[name]), name


def test_selector_steps_against_oracle(torch_gpu):
    torch = torch_gpu
    w = World(torch, seed=31)
    say("case selector step A (prefill only)")
    reqs = [(1, "a", 4100, 30, False), (2, "b", 4990, 10, False), (3, "c", 5990, 20, False), (5, "e", 0, 25, False)]
    out, state, host = w.step(reqs)
    assert tuple(out.shape) == (85, 1, TOPK)
    w.oracle_ingest(state, host, True)
    w.check_state(state)
    rows = out[:, 0].cpu().numpy()
    got_keys = w.indexer.prefill.score_keys[:85].cpu().numpy().view(np.uint16)
    vis = w.indexer.prefill.row_valid[:85].cpu().numpy()
    for r in range(85):
        assert np.array_equal(rows[r], li.topk_reference(got_keys[r], int(vis[r]))), r
    w.check_prefill_rows(rows, host, [(i, rows[p.begin:p.stop]) for i, p in enumerate(host.plans)])
    assert w.imported == {1, 2, 3, 5} and w.storage.imported == {1, 2, 3, 5}

    say("case selector step B (decode only, MTP rows, one empty request row)")
    reqs = [(2, "b", 5000, 4, True), (1, "a", 4130, 1, True), (3, "c", 6010, 3, True)]
    out, state, host = w.step(reqs)
    assert tuple(out.shape) == (8, 1, TOPK)
    meta, ends = w.oracle_ingest(state, host, False)
    w.check_decode(state, host, meta, ends, out[:, 0].cpu().numpy())
    w.check_state(state)

    say("case selector step C (mixed)")
    reqs = [(2, "b", 5004, 2, True), (4, "d", 3000, 12, False), (1, "a", 4131, 1, True), (3, "c", 6013, 20, False)]
    out, state, host = w.step(reqs)
    assert tuple(out.shape) == (35, 1, TOPK)
    w.oracle_ingest(state, host, True)
    # The decode rows' packing as the selector prepared it.
    dec = [p for p in host.plans if p.decode]
    meta = ad.prepare_metadata(B, [p.stop - p.begin for p in dec], [p.begin for p in dec], [p.owner for p in dec])
    ends = ad.bind_positions(meta, host.positions)
    rows = out[:, 0].cpu().numpy()
    decode_rows = np.concatenate([rows[p.begin:p.stop] for p in dec])
    w.check_decode(state, host, meta, ends, decode_rows)
    w.check_state(state)
    w.check_prefill_rows(rows, host, [(i, rows[p.begin:p.stop]) for i, p in enumerate(host.plans) if not p.decode])
    assert w.storage.imported == {1, 2, 3, 4, 5}


def test_selector_tail_source_against_oracle(torch_gpu):
    """The selector copies `tail_source` (columns 2:4 of [batch, 4] ABC descriptors, as the
    reference's binding slices them) into the update's tail bounds before each decode
    forward: a tail of recent positions shorter than the ring, one longer than the ring
    inside the hot range, an empty one. Decode outputs against the oracle's round with the
    same tails."""
    torch = torch_gpu
    ring = 384
    w = World(torch, seed=41, ring=ring)
    say("case selector tail: prefill")
    w.step([(1, "a", 4100, 30, False), (2, "b", 4990, 10, False), (3, "c", 5990, 20, False)])
    descriptors = torch.zeros((B, 4), dtype=torch.int32, device="cuda")
    w.selector.tail_source = descriptors[:, 2:4]
    for step, reqs in enumerate([[(2, "b", 5000, 4, True), (1, "a", 4130, 1, True), (3, "c", 6010, 3, True)],
                                 [(2, "b", 5004, 2, True), (1, "a", 4131, 1, True), (3, "c", 6013, 1, True)]]):
        say(f"case selector tail: decode step {step}")
        ends = [start + count for _, _, start, count, _ in reqs]
        tails = np.array([[ends[0] - 300, ends[0]], [1000, 1500], [0, 0], [0, 0]], np.int32)
        descriptors[:, 2:4].copy_(torch.from_numpy(tails))
        w.h_tail = tails
        out, state, host = w.step(reqs)
        assert np.array_equal(w.tail.cpu().numpy(), tails)
        meta, q_ends = w.oracle_ingest(state, host, False)
        w.check_decode(state, host, meta, q_ends, out[:, 0].cpu().numpy())
        w.check_state(state)
        so = w.update.slot_output[:, 0].cpu().numpy()
        assert (so >= RESIDENT).any()  # some selections resolved to ring slots


def test_selector_rejects_unbound_inputs(torch_gpu):
    torch = torch_gpu
    w = World(torch, seed=5)
    s = w.storage
    with pytest.raises(RuntimeError, match="needs a selection"):
        w.selector.slots(1)
    other = kvip_amd.QueryInputs(torch, B, "cuda", history=HISTORY)
    with pytest.raises(ValueError, match="not the packed QueryInputs buffer"):
        kvip_amd.VllmIndexSelector(torch, inputs=other, rotating=w.rot, update=w.update, logical_ids=s.logical_ids,
                                   row_owners=other.row_owners)
    with pytest.raises(ValueError, match="row owners"):
        kvip_amd.VllmIndexSelector(torch, inputs=w.inputs, rotating=w.rot, update=w.update,
                                   logical_ids=s.logical_ids, row_owners=w.inputs.row_owners[:2])
    with pytest.raises(ValueError, match="share an owner row"):
        sel = kvip_amd.VllmIndexSelector(torch, inputs=w.inputs, rotating=w.rot, update=w.update,
                                         logical_ids=s.logical_ids, row_owners=w.inputs.row_owners,
                                         unique_active_owners=True)
        sel.prepare([kvip_amd.RequestPlan(1, "x", 0, 1), kvip_amd.RequestPlan(1, "y", 1, 2)])
