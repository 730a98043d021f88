"""GPU parity at the benchmark configurations' own shapes, through the C ABI.

C1  batch 4, ctx 4096, bf16 Q/K, fp32 weights, no scales (the bench's c1 workload): the
    decode forward end to end. Every row scored by the oracle (1e-2 relative, > 99 %
    identical keys), TopK bit-exact against the oracle's TopK of the GPU's keys and inside
    the oracle's one-ulp cutoff band; the GPU TopK fed the oracle's own keys bit-exact
    against the oracle's TopK; the gather byte-exact.
C2  batch 64, ctx U[8192, 32768], fp8 (the bench workload, same seed): the decode forward;
    every row's TopK bit-exact against the oracle's TopK of the GPU's keys, both single pass
    and in the reference's trunk-merge order for this batch (trunk 8192: more than 16
    requests, indexer_vector.h:375-379 with indexer.h:193-196); the rows with ctx in
    (24576, 32768] scored by the oracle (3e-2 relative, > 99 % identical keys) with their
    TopK inside the oracle's one-ulp cutoff band; the gather byte-exact for every row.
C3  one sequence, 4096 query rows x 65536 keys, right-down causal: row_valid against the
    closed form, the histogram totals of every row, 16 sampled rows (first, middle, last
    of the causal range) scored by the oracle, TopK of every row bit-exact on the GPU keys
    and inside the cutoff band on the sampled rows, and the Index update of the 4096 new
    rows byte-exact.

Bars as in tests/test_gpu_lifetch.py and tests/test_gpu_prefill.py (written in each test)."""
import numpy as np
import pytest

import kvip_amd
from kvip_amd import synthetic
from oracle import indexer as ref

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)


def fp8_host(torch, t):
    return ref.fp8_e4m3_decode(t.view(torch.uint8).cpu().numpy())


def rows_of_pages(torch, cache, table_row, count):
    """Host float32 rows [count, ...] of a paged device cache through one block-table row."""
    pages = torch.from_numpy(np.asarray(table_row[:(count + 127) // 128], np.int64)).to(cache.device)
    part = cache[pages]
    host = fp8_host(torch, part) if part.dtype == torch.float8_e4m3fn else part.cpu().numpy()
    return host.reshape((-1,) + tuple(host.shape[2:]))[:count]


def assert_close_row(got, want, rtol, what):
    g = ref.score_values(got).astype(np.float64)
    w = ref.score_values(want).astype(np.float64)
    bad = np.abs(g - w) > rtol * np.abs(w) + rtol * np.abs(w).max()
    assert not bad.any(), f"{what}: {int(bad.sum())} scores outside rtol {rtol}"


def test_c1_end_to_end_against_oracle(torch_gpu):
    torch = torch_gpu
    import ctypes
    from kvip_amd.runtime import abi

    say("case C1 batch 4 ctx 4096 bf16 (bench c1 workload)")
    wl = synthetic.config_workload(torch, "c1", "cuda", seed=2026)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    keys = rot.score_keys.cpu().numpy().view(np.uint16)
    topk = rot.topk.cpu().numpy()
    table = wl.block_table.cpu().numpy()
    q = wl.query.float().cpu().numpy()
    w = wl.weights.float().cpu().numpy()
    want_keys = np.zeros_like(keys)
    for r, v in enumerate(wl.ctx):
        v = int(v)
        k = rows_of_pages(torch, wl.keys.float(), table[r], v)
        want = ref.li_keys(q[r], k, w[r], None, None)
        want_keys[r, :v] = want
        assert_close_row(keys[r, :v], want, 1e-2, f"row {r}")
        assert np.array_equal(topk[r], ref.topk_reference(keys[r], v)), r
        assert ref.validate_topk_band(topk[r], ref.score_values(want)), r
    same = ref.identical_share(keys, want_keys, [int(v) for v in wl.ctx])
    say(f"  identical keys: {same:.5f}")
    assert same > 0.99
    say("  gather of the 4 rows")
    assert np.array_equal(upd.output.cpu().numpy(), ref.fetch_gather(wl.kv_cache.cpu().numpy(), table, topk))
    say("  TopK fed the oracle's keys")
    rot.score_keys.copy_(torch.from_numpy(want_keys.view(np.int16)))
    rot.topk.fill_(-5)
    args = rot.topk_args(use_histogram=False)
    abi.check(abi.load_library().kvip_hip_topk(ctypes.byref(args), abi.stream_handle(torch, rot.device)), "topk")
    torch.cuda.synchronize()
    got = rot.topk.cpu().numpy()
    for r, v in enumerate(wl.ctx):
        assert np.array_equal(got[r], ref.topk_reference(want_keys[r], int(v))), r
    assert int(rot.status.item()) == 0


def test_c2_full_shape_against_oracle(torch_gpu):
    torch = torch_gpu
    say("case C2 batch 64 ctx U[8192,32768] fp8 (bench seed 2026)")
    wl = synthetic.config_workload(torch, "c2", "cuda", seed=2026)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    keys = rot.score_keys.cpu().numpy().view(np.uint16)
    topk = rot.topk.cpu().numpy()
    ctx = wl.ctx
    say("  TopK of all 64 rows against the oracle (single pass and trunk 8192)")
    for r, v in enumerate(ctx):
        want = ref.topk_reference(keys[r], int(v), trunk=8192)
        assert np.array_equal(topk[r], want), r
        assert np.array_equal(topk[r], ref.topk_reference(keys[r], int(v))), r
    long_rows = [r for r, v in enumerate(ctx) if v > 24576]
    assert len(long_rows) >= 8, ctx
    table = wl.block_table.cpu().numpy()
    q = fp8_host(torch, wl.query)
    w = wl.weights.float().cpu().numpy()
    same = total = 0
    for r in long_rows[:12]:
        v = int(ctx[r])
        say(f"  oracle scores of row {r} (ctx {v})")
        k = rows_of_pages(torch, wl.keys, table[r], v)
        ks = rows_of_pages(torch, wl.key_scale, table[r], v)
        want = ref.li_keys(q[r], k, w[r], None, ks)
        assert_close_row(keys[r, :v], want, 3e-2, f"row {r}")
        share_keys = np.zeros((1, v), np.uint16)
        share_keys[0] = keys[r, :v]
        n = ref.identical_share(share_keys, want[None, :], [v])
        same += n * v
        total += v
        assert ref.validate_topk_band(topk[r], ref.score_values(want)), r
    say(f"  identical keys on the long rows: {same / total:.5f}")
    assert same / total > 0.99
    say("  gather of all 64 rows")
    kv = wl.kv_cache.cpu().numpy()
    assert np.array_equal(upd.output.cpu().numpy(), ref.fetch_gather(kv, table, topk))


def test_c3_full_shape_against_oracle(torch_gpu):
    torch = torch_gpu
    from types import SimpleNamespace as NS
    from kvip_amd.adapters.vllm.index_import import VllmIndexCacheStorage

    say("case C3 prefill 4096 x 65536 causal fp8")
    wl = synthetic.prefill_workload(torch, "cuda", seed=2026)
    q_len, k_len, heads = wl["q_len"], wl["k_len"], wl["heads"]
    idx = kvip_amd.PrefillIndexer(torch, max_rows=q_len, max_context=k_len, max_sequences=1, device="cuda",
                                  heads=heads)
    idx.bind(wl["query"], wl["weights"], wl["query_scale"], wl["keys"], wl["key_scale"], wl["cu_seqlens_q"],
             wl["seq_lens_k"], wl["block_table"])
    idx.score()
    torch.cuda.synchronize()
    assert int(idx.status.item()) == 0
    vis = ref.prefill_visible([0, q_len], [k_len])
    assert np.array_equal(idx.row_valid[:q_len].cpu().numpy(), vis)
    hist = idx.histogram[:q_len].cpu().numpy().astype(np.int64)
    assert np.array_equal(hist.sum(axis=1), vis)
    keys = idx.score_keys[:q_len].cpu().numpy().view(np.uint16)
    for r in (0, 2047, 4095):
        assert np.array_equal(hist[r], np.bincount(keys[r, :vis[r]] >> 8, minlength=256)), r
    top = idx.select().cpu().numpy()
    torch.cuda.synchronize()
    assert int(idx.status.item()) == 0 and not idx.histogram.any()
    say("  TopK of all 4096 rows against the oracle's TopK of the GPU keys")
    for r in range(q_len):
        assert np.array_equal(top[r], ref.topk_reference(keys[r], int(vis[r]))), r
    sample = sorted(set([0, 1, 2, 1023, 1024, 2047, 2048, 2049, 3000, 3071, 3584, 4000, 4093, 4094, 4095, 511]))
    table = wl["block_table"].cpu().numpy()[0]
    k_all = rows_of_pages(torch, wl["keys"], table, k_len)
    ks_all = rows_of_pages(torch, wl["key_scale"], table, k_len)
    q = fp8_host(torch, wl["query"])
    w = wl["weights"].cpu().numpy()
    qs = wl["query_scale"].cpu().numpy()
    want = np.zeros((len(sample), k_len), np.uint16)
    for i, r in enumerate(sample):
        v = int(vis[r])
        say(f"  oracle scores of row {r} (visible {v})")
        want[i, :v] = ref.li_keys(q[r], k_all[:v], w[r], qs[r], ks_all[:v])
        assert_close_row(keys[r, :v], want[i, :v], 3e-2, f"row {r}")
        assert ref.validate_topk_band(top[r], ref.score_values(want[i, :v])), r
    same = ref.identical_share(keys[sample], want, vis[sample])
    say(f"  identical keys on the sampled rows: {same:.5f}")
    assert same > 0.99
    say("  Index update of the 4096 new rows")
    storage = VllmIndexCacheStorage(torch, 1, k_len, 2048, "cuda")
    plan = NS(owner=0, request="c3", start=k_len - q_len, begin=0, stop=q_len)
    storage.prepare([plan])
    cache = (wl["keys"].view(-1, 128, 1, 128), wl["key_scale"].view(-1, 128, 1))
    metadata = NS(block_size=128, block_table=wl["block_table"], slot_mapping=wl["slot_mapping"])
    storage.ingest_prefill(cache, metadata, [plan], wl["positions"])
    torch.cuda.synchronize()
    assert int(storage.status.item()) == 0
    src = wl["keys"].view(torch.uint8).view(-1, 128).cpu().numpy()
    src_s = wl["key_scale"].view(-1).cpu().numpy()
    slots = wl["slot_mapping"].cpu().numpy()
    dst = storage.keys.view(torch.uint8).view(-1, 128).cpu().numpy()
    dst_s = storage.scales.view(-1).cpu().numpy()
    pos = wl["positions"].cpu().numpy()
    assert np.array_equal(dst[pos], src[slots])
    assert np.array_equal(dst_s[pos], src_s[slots])
    prefix = np.arange(k_len - q_len)
    prefix_slots = table[prefix // 128].astype(np.int64) * 128 + prefix % 128
    assert np.array_equal(dst[prefix], src[prefix_slots])
    assert np.array_equal(dst_s[prefix], src_s[prefix_slots])


class ResidentMirror:
    """Host copies of a resident update's tables, advanced by oracle.resident.resident_round
    request by request, plus one oracle SlotLRU per request committing the slot outputs."""

    def __init__(self, torch, upd, capacity):
        from oracle import cache as lru_ref

        t = torch
        self.torch, self.upd = torch, upd
        self.keys = upd.keys.view(t.uint8).cpu().numpy()
        self.scales = upd.scales.cpu().numpy()
        self.addresses = upd.addresses.cpu().numpy()
        self.logical = upd.logical_ids.cpu().numpy()
        self.valid = upd.hot_valid.cpu().numpy()
        self.hot = upd.hot_cache.cpu().numpy()
        self.pool = upd.host_pool.numpy()
        self.owners = upd.row_owners.cpu().numpy()
        self.lrus = []
        for _ in range(upd.rotating.batch):
            lru = lru_ref.SlotLRU()
            lru.resize(capacity, capacity)
            self.lrus.append(lru)

    def round(self, selected):
        """Oracle round on TopK rows [batch * q, 2048] with the mirrored LRU candidates."""
        from oracle import resident as rs

        upd = self.upd
        q = upd.rotating.rows_per_request
        outs = []
        for b, o in enumerate(self.owners):
            cand = self.lrus[b].slots.astype(np.int64)
            reserved = rs.reserved_from_candidates(cand, upd.resident)
            lout, sout, res, err = rs.resident_round(
                selected[b * q:(b + 1) * q].astype(np.int64), upd.history, upd.resident, self.keys[o],
                self.scales[o], self.addresses[o], self.logical[o], self.valid[o], reserved, cand, self.hot[o],
                self.pool)
            outs.append((lout, sout, res, err, cand))
        return outs

    def compare(self, outs, lru_slots_before):
        t, upd = self.torch, self.upd
        q = upd.rotating.rows_per_request
        lo = upd.logical_output.cpu().numpy().reshape(len(outs), q, 2048)
        so = upd.slot_output.cpu().numpy().reshape(len(outs), q, 2048)
        counts = upd.miss_counts.cpu().numpy()
        status = upd.status.cpu().numpy()
        for b, (lout, sout, res, err, cand) in enumerate(outs):
            assert np.array_equal(lru_slots_before[b], cand), f"candidates of request {b}"
            assert status[b] == err, (b, status[b], err)
            assert np.array_equal(lo[b], lout), b
            assert np.array_equal(so[b], sout), b
            added = list(res["added"]) + [0] * (4 - len(res["added"]))
            assert counts[b].tolist() == added + [int(res["added"].sum())], b
        assert np.array_equal(upd.keys.view(t.uint8).cpu().numpy(), self.keys)
        assert np.array_equal(upd.scales.cpu().numpy(), self.scales)
        assert np.array_equal(upd.addresses.cpu().numpy(), self.addresses)
        assert np.array_equal(upd.logical_ids.cpu().numpy(), self.logical)
        assert np.array_equal(upd.hot_valid.cpu().numpy(), self.valid)
        assert np.array_equal(upd.hot_cache.cpu().numpy(), self.hot)
        for b, (lout, sout, res, err, cand) in enumerate(outs):
            self.lrus[b].commit(sout.reshape(-1))
        return int(counts[:, 4].sum())


def test_c4_full_shape_against_oracle(torch_gpu):
    """C4: 16 requests, history 131072, 16384 hot slots, misses from the pinned host pool;
    two rounds on TopK rows drawn ~80 % hot under Zipf(1.1) popularity, then one full
    forward (LI over 16 x 131072 Index rows, TopK, round); the device LRU chains commit
    every round and feed the next one's candidates. Every output, count, table and the
    candidates bit-exact against the oracle after every round."""
    import ctypes
    from kvip_amd.runtime import abi

    torch = torch_gpu
    batch, history, resident = 16, 131072, 16384
    say("case C4 16 x 131072, resident 16384 (filling the host pool)")
    rot, upd, fwd = synthetic.resident_workload(torch, kvip_amd, "cuda", seed=44, batch=batch, history=history,
                                                resident=resident, fill_pool=True)
    lru = kvip_amd.SlotLRUChains(torch, batch, resident, "cuda", slots=upd.lru_slots)
    torch.cuda.synchronize()
    mirror = ResidentMirror(torch, upd, resident)
    lib = abi.load_library()
    picks = synthetic.resident_selections(torch, np.random.default_rng(44), steps=2, batch=batch, q_rows=1,
                                          history=history, resident=resident)
    commit_rows = upd.slot_output.view(batch, -1)
    for step in range(2):
        say(f"  round {step} on drawn TopK rows")
        before = upd.lru_slots.cpu().numpy()
        rot.topk.copy_(torch.from_numpy(picks[step]))
        abi.check(lib.kvip_hip_resident_round(ctypes.byref(upd.args), abi.stream_handle(torch, rot.device)), "round")
        lru.commit(commit_rows)
        torch.cuda.synchronize()
        outs = mirror.round(picks[step])
        misses = mirror.compare(outs, before)
        say(f"    misses {misses} of {batch * 2048} ({1 - misses / (batch * 2048):.3f} hits)")
        assert not upd.status.any()
    say("  full forward: LI over 16 x 131072, TopK, round")
    before = upd.lru_slots.cpu().numpy()
    fwd()
    lru.commit(commit_rows)
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    keys = rot.score_keys.cpu().numpy().view(np.uint16)
    topk = rot.topk.cpu().numpy()
    for r in range(batch):
        assert np.array_equal(topk[r], ref.topk_reference(keys[r], history, trunk=16384)), r
    q = fp8_host(torch, rot.query)
    w = rot.weights.float().cpu().numpy()
    for r in (0, 11):
        say(f"    oracle scores of row {r} over the Index rows of owner {r}")
        k = ref.fp8_e4m3_decode(mirror.keys[r])
        want = ref.li_keys(q[r], k, w[r], None, mirror.scales[r])
        assert_close_row(keys[r, :history], want, 3e-2, f"row {r}")
        assert ref.validate_topk_band(topk[r], ref.score_values(want)), r
    outs = mirror.round(topk)
    mirror.compare(outs, before)


def test_c5_full_shape_graph_against_oracle(torch_gpu):
    """C5: 32 decode requests (ctx U[4096, 65536], resident 16384, misses from the pinned
    host pool, LRU chains committed inside the round) + prefill chunks of 2048 and 1536
    rows, one hipGraph replayed twice. After each replay: the ingest of every new token
    byte-exact; decode TopK bit-exact on the GPU keys for all 32 rows, 6 rows scored by the
    oracle inside the cutoff band; the resident round, its tables and the LRU candidates
    bit-exact against the oracle on the device TopK; prefill row_valid against the closed
    form, TopK of every row bit-exact on the GPU keys, 16 rows scored by the oracle."""
    torch = torch_gpu
    say("case C5 32 decode + 2048/1536 prefill, one hipGraph (filling the host pool)")
    wl = synthetic.mixed_workload(torch, kvip_amd, "cuda", seed=2026, lru=True, fill_pool=True)
    upd, rot, pf = wl.update, wl.rot, wl.prefill
    # One eager round first (every kernel loaded before the capture); the LRU chains then
    # restart cold and the mirror takes the state from there.
    wl.round()
    wl.lru.reset(wl.resident)
    torch.cuda.synchronize()
    mirror = ResidentMirror(torch, upd, wl.resident)
    cache_k = wl.cache_keys.view(torch.uint8).view(-1, 128).cpu().numpy()
    cache_s = wl.cache_scales.view(-1).cpu().numpy()
    src, dst = np.asarray(wl.sources), np.asarray(wl.targets)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            wl.round()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    nd = len(wl.decode_ctx)
    q = fp8_host(torch, rot.query)
    w = rot.weights.float().cpu().numpy()
    qs = None if rot.query_scale is None else rot.query_scale.cpu().numpy()
    for replay in range(2):
        say(f"  replay {replay}")
        before = upd.lru_slots.cpu().numpy()
        graph.replay()
        torch.cuda.synchronize()
        for st in (upd.status, rot.status, pf.status, wl.round.status):
            assert not st.any(), st
        # Ingest on the mirror (the round's first stage).
        flat_k = mirror.keys.reshape(-1, 128)
        flat_s = mirror.scales.reshape(-1)
        flat_k[dst] = cache_k[src]
        flat_s[dst] = cache_s[src]
        keys = rot.score_keys.cpu().numpy().view(np.uint16)
        topk = rot.topk.cpu().numpy()
        for b, c in enumerate(wl.decode_ctx):
            assert np.array_equal(topk[b], ref.topk_reference(keys[b], int(c))), b
        for b in (0, 7, 15, 23, 31, int(np.argmax(wl.decode_ctx))):
            c = int(wl.decode_ctx[b])
            want = ref.li_keys(q[b], ref.fp8_e4m3_decode(mirror.keys[b, :c]), w[b], None if qs is None else qs[b],
                               mirror.scales[b, :c])
            assert_close_row(keys[b, :c], want, 3e-2, f"decode row {b}")
            assert ref.validate_topk_band(topk[b], ref.score_values(want)), b
        outs = mirror.round(topk)
        misses = mirror.compare(outs, before)
        say(f"    decode misses {misses} of {nd * 2048}")
        # Prefill chunks on the paged cache.
        rows = sum(qq for qq, _ in wl.chunks)
        vis = ref.prefill_visible(wl.cu.cpu().numpy(), wl.kl.cpu().numpy())
        assert np.array_equal(pf.row_valid[:rows].cpu().numpy(), vis)
        pkeys = pf.score_keys[:rows].cpu().numpy().view(np.uint16)
        ptop = pf.topk[:rows].cpu().numpy()
        for r in range(rows):
            assert np.array_equal(ptop[r], ref.topk_reference(pkeys[r], int(vis[r]))), r
        if replay == 0:
            table = wl.table.cpu().numpy()
            pq = fp8_host(torch, wl.pf_query)
            pw = wl.pf_weights.cpu().numpy()
            pqs = wl.pf_qscale.cpu().numpy()
            cu = wl.cu.cpu().numpy()
            for s, (q_len, k_len) in enumerate(wl.chunks):
                k_all = rows_of_pages(torch, wl.cache_keys, table[s], k_len)
                ks_all = rows_of_pages(torch, wl.cache_scales, table[s], k_len)
                for j in sorted(set([0, 1, q_len // 2, q_len - 2, q_len - 1, q_len // 3, 2 * q_len // 3, 5])):
                    r = int(cu[s]) + j
                    v = int(vis[r])
                    want = ref.li_keys(pq[r], k_all[:v], pw[r], pqs[r], ks_all[:v])
                    assert_close_row(pkeys[r, :v], want, 3e-2, f"prefill row {r}")
                    if v >= 2048:
                        assert ref.validate_topk_band(ptop[r], ref.score_values(want)), r
