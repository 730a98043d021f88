"""Decode LI+TopK+Fetch throughput on one MI355X (config 2 by default).

One step = one decode round of the hot path over one batch of synthetic input that
is already resident in HBM: lightning-indexer scoring of every context token of the
64 requests, TopK-2048 per request, and the Fetch gather of the 2048 selected
656-byte KV rows per request into a contiguous [64, 2048, 656] buffer. Rounds run as
kernel nodes of captured hipGraphs, 8 rounds per graph by default (--rounds-per-graph;
graph_ms_per_step reports one graph launch per round beside it).

Prints one JSON line (rank 0): queries/s, per-kernel HIP-event timings, the roofline
of the dominant kernel against MI355X's 8 TB/s HBM peak, the CPU baseline (the
oracle timed on a bounded sample of the same workload on this host) and, under
"lidu", the device time of one kvip.lidu resolver call at the config-4 shape.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP8_MFMA_PEAK_TFLOPS = 5000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
TOPK = 2048
# Rounds captured back to back in one hipGraph by the resident and mixed legs.
CURSOR_ROUNDS_PER_GRAPH = 4


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default="c2", choices=["c1", "c2"])
    p.add_argument("--rounds-per-graph", type=int, default=8,
                   help="decode rounds captured back to back in one hipGraph (as inside a model's decode "
                        "graph); 1 = one graph launch per round; 1 or even")
    p.add_argument("--seed", type=int, default=2026)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-mtp", action="store_true", help="skip the 4-rows-per-request (MTP) decode leg")
    p.add_argument("--no-lidu", action="store_true", help="skip the kvip.lidu timing leg")
    p.add_argument("--no-resident", action="store_true", help="skip the resident-cache round timing leg")
    p.add_argument("--no-prefill", action="store_true", help="skip the config-3 prefill timing leg")
    p.add_argument("--no-mixed", action="store_true", help="skip the config-5 mixed-round timing leg")
    p.add_argument("--no-sfa", action="store_true", help="skip the sparse-attention consumer timing leg")
    p.add_argument("--only", default=None,
                   help="run just this leg (mtp, lidu, resident, cache_ops, prefill, mixed, sfa) and print its JSON "
                        "(profiling runs; no headline line)")
    p.add_argument("--sequential", action="store_true",
                   help="resident and mixed legs on one stream (Fetch after the Index update, prefill after the "
                        "decode; no speculative-prefetch loop): each kernel runs alone, for per-kernel profiles")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a plain 1 GiB device copy (for rocprof FETCH/WRITE_SIZE scaling)")
    return p.parse_args()


def algorithmic_bytes(wl, heads, has_qscale):
    """Per-kernel algorithmic HBM bytes of one step (score materialisation excluded)."""
    ctx = wl.ctx.astype(np.int64)
    rows = len(ctx) * wl.rows_per_request
    elem = 1 if wl.query.element_size() == 1 else 2
    key_bytes = 128 * elem + (4 if wl.key_scale is not None else 0)
    score = int((ctx * key_bytes).sum() + (4 * ((ctx + 127) // 128)).sum())
    score += rows * (heads * 128 * elem + heads * wl.weights.element_size() + (heads * 4 if has_qscale else 0))
    row_bytes = int(wl.kv_cache.shape[2])
    live = np.minimum(ctx, TOPK).repeat(wl.rows_per_request)
    topk = rows * TOPK * 4
    gather = int(live.sum()) * row_bytes * 2
    return {"indexer": score, "topk": topk, "fetch": gather}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary, when it was taken on the current sources of the measured kernels (the files it
    lists); otherwise None."""
    from kvip_amd.runtime.build import files_digest

    path = ROOT / "profiles" / "decode_c2_traffic.json"
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if not data.get("sources") or data.get("source_digest") != files_digest(data["sources"]):
        return None
    return data.get("traffic_bytes", {}).get(kernel)


def cpu_baseline(torch, wl, rot, budget_s):
    """The torch-CPU restatement (oracle/cpu_torch.py) of one decode query row, timed on the
    host over the rows of the same workload until the time budget is spent: decode the fp8
    Q/K bytes to float32, LI keys (two threaded BLAS products), TopK-2048, Fetch gather.
    Threads: os.cpu_count() as planned, capped by this process's CPU affinity and by
    OMP_NUM_THREADS when set (the CPU share a job gets on a shared host)."""
    from oracle import cpu_torch

    logical = os.cpu_count() or 1
    threads = min(logical, len(os.sched_getaffinity(0)))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, max(int(os.environ["OMP_NUM_THREADS"]), 1))
    try:
        import psutil

        physical = psutil.cpu_count(logical=False)
    except Exception:  # noqa: BLE001 - informational only
        physical = None
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        table = wl.block_table.cpu()
        kv_rows = wl.kv_cache.cpu().reshape(-1, int(wl.kv_cache.shape[2]))
        staged = []  # per request: fp8 Q/K bytes and scales on the host (staging, untimed)
        for b in range(wl.batch):
            v = int(wl.ctx[b])
            pages = table[b, :(v + 127) // 128]
            k_raw = wl.keys[pages.to(wl.keys.device).long()].view(torch.uint8).reshape(-1, 128)[:v].cpu()
            ks = None if wl.key_scale is None else wl.key_scale[pages.to(wl.keys.device).long()].reshape(-1)[:v].cpu()
            qs = None if wl.query_scale is None else wl.query_scale[b].float().cpu()
            staged.append((wl.query[b].view(torch.uint8).cpu(), k_raw, wl.weights[b].float().cpu(), qs, ks, pages, v))
        cpu_torch.decode_row(torch, *staged[0][:5], kv_rows, staged[0][5], staged[0][6])  # warm-up
        done, elapsed, nbytes = 0, 0.0, 0
        while elapsed < budget_s:
            q, k, w, qs, ks, pages, v = staged[done % len(staged)]
            t0 = time.perf_counter()
            cpu_torch.decode_row(torch, q, k, w, qs, ks, kv_rows, pages, v)
            elapsed += time.perf_counter() - t0
            nbytes += v * (128 + (4 if ks is not None else 0)) + 4 * ((v + 127) // 128) + 2 * TOPK * kv_rows.shape[1]
            done += 1
    finally:
        torch.set_num_threads(saved)
    return {"value": round(done / elapsed, 3), "unit": "queries/s", "cores": threads, "kind": "port",
            "physical_cores": physical, "logical_cpus": logical, "gbs": round(nbytes / elapsed / 1e9, 2),
            "sample": f"{done} query rows cycling over the {len(staged)} requests of the same workload, "
                      f"{elapsed:.1f} s: torch-CPU restatement (fp8 decode, float32 BLAS dot products and head "
                      f"reduction, bf16 keys, TopK-2048, 656-byte row gather) on {threads} torch threads; host "
                      f"has {physical} physical cores, {logical} logical CPUs"}


def lidu_leg(torch, kvip_amd, device, seed, iters=50, reps=7):
    """Device time of one kvip.lidu call at the config-4 shape (16 MTP requests x
    4 query rows, resident budget 16384 of a 131072-token history, ~80 % hits). Each call
    must start from the same maps, so two graphs are replayed back to back `iters` times:
    one restores the maps, the other restores them and runs lidu; the difference of the
    two (medians over `reps` alternations) is lidu's time with host launch latency hidden
    behind the queued replays."""
    from kvip_amd import synthetic

    dev, outs, args = synthetic.lidu_workload(torch, device, seed=seed)
    names = ("token_to_slot_pool", "slot_to_token_pool", "eviction_cursors")
    saved = {k: dev[k].clone() for k in names}

    def restore():
        for k in names:
            dev[k].copy_(saved[k])

    kvip_amd.lidu(*args)  # allocates the per-batch workspace before capture
    torch.cuda.synchronize()
    graphs = []
    for body in (restore, lambda: (restore(), kvip_amd.lidu(*args))):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body()
        graphs.append(g)
    def timed(g):
        for _ in range(3):
            g.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            g.replay()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) * 1e3 / iters

    # The two graphs alternate `reps` times; the medians damp clock and queue drift.
    samples = [[], []]
    for _ in range(reps):
        for k, g in enumerate(graphs):
            samples[k].append(timed(g))
    times = [float(np.median(x)) for x in samples]
    counts = outs["miss_counts"].cpu().numpy()
    if (counts[:-1] < 0).any():
        raise RuntimeError(f"lidu rejected a request: {counts.tolist()}")
    return {"workload": "c4 shape: 16 requests x 4 MTP rows, budget 16384, history 131072, ~80% hits",
            "us_per_call": round(times[1] - times[0], 2), "restore_us": round(times[0], 2),
            "unique_misses_per_request": round(float(counts[:-1].mean()), 1), "calls": iters * reps}


def _query_walk(torch, base, sets, seed, step=0.3):
    """uint8 view [sets, *base.shape] of fp8 query sets along a random walk (set 0 is the
    base, set k = sqrt(1 - step^2) * set k-1 + step * N(0, 1)): consecutive rounds select
    overlapping but drifting positions, as consecutive decode steps do."""
    from kvip_amd import synthetic

    gen = torch.Generator(device=base.device)
    gen.manual_seed(seed)
    vals = base.float()
    out = torch.empty((sets, *base.shape), dtype=torch.uint8, device=base.device)
    out[0].copy_(base.view(torch.uint8))
    for k in range(1, sets):
        vals = (1.0 - step * step) ** 0.5 * vals + step * torch.randn(vals.shape, generator=gen, device=base.device)
        out[k].copy_(synthetic.saturating_fp8(torch, vals).view(torch.uint8))
    return out


def _cursor_rounds(torch, body, warm, rounds, sets, per_graph=None, label="rounds"):
    """Consecutive rounds from one captured hipGraph of `per_graph` rounds: body(cursor)
    enqueues round `cursor` (a device int64 [1] that the graph then advances), reading that
    round's inputs and recording its outcome by device indexing. One eager round on a side
    stream (code-object loading), cursor reset, capture; warm / per_graph untimed replays,
    then rounds / per_graph back-to-back replays timed with HIP events on the launch stream
    (the rounds of a graph follow each other with no host launch between them, as a model's
    layers do inside its captured decode step); the cursor stays below `sets`, the number of
    input sets the body indexes. Prints a progress line (`label`) to stderr. Returns us per
    round."""
    per_graph = CURSOR_ROUNDS_PER_GRAPH if per_graph is None else per_graph
    if warm + rounds > sets:
        raise ValueError(f"{warm} + {rounds} rounds need as many input sets (have {sets})")
    if warm % per_graph or rounds % per_graph:
        raise ValueError(f"warm-up ({warm}) and timed rounds ({rounds}) must be multiples of {per_graph}")
    stream = torch.cuda.current_stream()
    cursor = torch.zeros(1, dtype=torch.int64, device=stream.device)

    def step():
        body(cursor)
        cursor.add_(1)

    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    cursor.zero_()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            step()
    cursor.zero_()
    torch.cuda.synchronize()
    for _ in range(warm // per_graph):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(rounds // per_graph):
        graph.replay()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / rounds
    print(f"bench: {label} loop done ({us:.1f} us per round)", file=sys.stderr, flush=True)
    return us


def _pick(torch, inputs, cursor, dst):
    """dst <- inputs[cursor] in one gather launch (dst is the bound input buffer)."""
    torch.index_select(inputs, 0, cursor, out=dst.view(1, *dst.shape))


def host_read_gbs(torch, device, nbytes=256 << 20):
    """Host-to-device bandwidth from pinned memory (one large copy): the ceiling of a Fetch
    whose rows live in a pinned host pool."""
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
    for _ in range(2):
        dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(4):
        dst.copy_(src, non_blocking=True)
    e1.record()
    e1.synchronize()
    return 4 * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9


def cache_ops_leg(torch, kvip_amd, device, seed, iters=20):
    """The per-step cache bookkeeping kernels alone, each captured 10 times in a hipGraph
    and replayed `iters` times (HIP events around the replays):
      update_abc:  one decode step of the ABC ring maps (python/kvip/cache/abc.py): 16
                   requests x 4 new tokens into a 2048-slot tail after 16384 history slots,
                   one layer;
      lru_commit:  SlotLRUChains.commit for 32 chains of 16384 slots with 2048 accessed slots
                   each (the C5 decode batch).
    Bytes are the arrays each kernel must read and write once."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out = {}
    history, tail, req, new = 16384, 2048, 16, 4
    t2s = torch.full((1, req, history + tail), -1, dtype=torch.int32, device=device)
    s2t = torch.full((1, req, history + tail), -1, dtype=torch.int32, device=device)
    begin = torch.randint(history, history + tail - new, (req,), generator=gen, device=device, dtype=torch.int32)
    desc = torch.stack([torch.zeros_like(begin), torch.arange(req, dtype=torch.int32, device=device), begin,
                        begin + new], dim=1)[None].contiguous()
    chains, cap = 32, 16384
    lru = kvip_amd.SlotLRUChains(torch, chains, cap, device)
    dest = torch.argsort(torch.rand((chains, cap), generator=gen, device=device), dim=1)[:, :TOPK]
    dest = dest.to(torch.int32).contiguous()
    calls = {"update_abc": (lambda: kvip_amd.update_abc(t2s, s2t, desc, req, history, tail),
                            req * (new * 4 * 2 + tail * 4 + 16)),
             "lru_commit": (lambda: lru.commit(dest), chains * (cap * 4 * 3 + TOPK * 4 + TOPK * 4))}
    stream = torch.cuda.current_stream()
    for name, (call, nbytes) in calls.items():
        call()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(10):
                call()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iters):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (iters * 10)
        out[name] = {"us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    out["workload"] = ("update_abc: 16 requests x 4 new tokens, tail 2048 after 16384 history slots; lru_commit: "
                       "32 chains x 16384 slots, 2048 accessed per chain")
    return out


def resident_leg(torch, kvip_amd, device, seed, rounds=24, warm=4, sequential=False):
    """config 4 on the resident cache: 16 requests, history 131072, 16384 hot
    slots, misses fetched from a pinned host pool, the device LRU chains (one per request)
    committed by every round inside the graph. Two loops of consecutive rounds, each a
    captured hipGraph of CURSOR_ROUNDS_PER_GRAPH rounds replayed back to back (HIP events
    around the timed replays), every round on inputs of its own (picked by a device cursor)
    and recording its misses:
      round:   the resident round alone (init, resolve, then the Fetch of the misses beside
               the Index update and LRU commit on a second stream) on TopK rows drawn ~80 %
               hot under Zipf(1.1) popularity, a fresh draw per round; timed again with the
               three stages in sequence on one stream (`sequential_us_per_round`);
      forward: the whole resident forward (LI over 16 x 131072 Index rows, TopK-2048, the
               round, LRU commit) on query sets along a random walk (consecutive rounds
               select overlapping, drifting positions).
    sequential: every loop on one stream (upd.overlap False) and no speculative-prefetch
    loop (its prefix TopK runs on a forked stream)."""
    from kvip_amd import synthetic

    batch, history, resident = 16, 131072, 16384
    n = warm + rounds + 1  # + the eager round before capture
    rot, upd, fwd = synthetic.resident_workload(torch, kvip_amd, device, seed=seed, batch=batch,
                                                history=history, resident=resident, overlap=not sequential)
    rng = np.random.default_rng(seed)
    picks = torch.from_numpy(synthetic.resident_selections(torch, rng, steps=n, batch=batch, q_rows=1,
                                                           history=history, resident=resident)).to(device)
    lru = kvip_amd.SlotLRUChains(torch, batch, resident, device, slots=upd.lru_slots)
    upd.attach_lru(lru)  # committed by every round right after its Index update
    trace = torch.zeros((n, batch), dtype=torch.int32, device=device)
    picks_now = [picks]

    def record(cursor):
        trace.index_copy_(0, cursor, upd.miss_counts[:, 4].view(1, batch))

    def round_body(cursor):
        _pick(torch, picks_now[0], cursor, rot.topk)
        upd.round()
        record(cursor)

    round_us = _cursor_rounds(torch, round_body, warm, rounds, n, label="resident round")
    if upd.status.any():
        raise RuntimeError(f"resident round failed: {upd.status.cpu().tolist()}")
    round_miss = trace[warm:warm + rounds].sum(1).float().mean().item()
    # The same loop with resolve, Fetch and Index update (+ LRU commit) in sequence on one
    # stream, on fresh draws of the same popularity (the cache continues from the loop above).
    picks_now[0] = torch.from_numpy(synthetic.resident_selections(
        torch, np.random.default_rng(seed + 1), steps=n, batch=batch, q_rows=1, history=history,
        resident=resident)).to(device)
    trace.zero_()
    upd.overlap = False
    seq_us = _cursor_rounds(torch, round_body, warm, rounds, n, label="resident round in sequence")
    upd.overlap = not sequential
    if upd.status.any():
        raise RuntimeError(f"resident round failed: {upd.status.cpu().tolist()}")
    seq_miss = trace[warm:warm + rounds].sum(1).float().mean().item()
    queries = _query_walk(torch, rot.query, n, seed)
    q_bytes = rot.query.view(torch.uint8)
    trace.zero_()

    def forward_body(cursor):
        _pick(torch, queries, cursor, q_bytes)
        fwd()
        record(cursor)

    fwd_us = _cursor_rounds(torch, forward_body, warm, rounds, n, label="resident forward")
    if upd.status.any() or rot.status.any():
        raise RuntimeError(f"resident forward failed: {upd.status.cpu().tolist()} {int(rot.status.item())}")
    fwd_miss = trace[warm:warm + rounds].sum(1).float().mean().item()
    out = {"workload": "c4 shape: 16 requests x 1 row, history 131072, resident 16384, misses fetched from pinned "
                       "host memory, LRU chains committed in the graph; round: TopK rows drawn ~80% hot (Zipf 1.1), "
                       "a fresh draw per round; forward: LI + TopK + round on query sets along a random walk",
           "us_per_round": round(round_us, 2), "misses_per_round": round(round_miss, 1),
           "sequential_us_per_round": round(seq_us, 2), "sequential_misses_per_round": round(seq_miss, 1),
           "hit_fraction": round(1.0 - round_miss / (batch * TOPK), 4),
           "fetch_gbs_lower_bound": round(round_miss * 656 / (round_us * 1e-6) / 1e9, 2),
           "forward_us": round(fwd_us, 2), "forward_misses_per_round": round(fwd_miss, 1),
           "forward_hit_fraction": round(1.0 - fwd_miss / (batch * TOPK), 4),
           "forward_index_gbs": round(batch * history * 132 / (fwd_us * 1e-6) / 1e9, 1), "rounds": rounds,
           "rounds_per_graph": CURSOR_ROUNDS_PER_GRAPH,
           "streams": "one" if sequential else "Fetch beside the Index update"}
    if sequential:
        return out
    del rot, upd, fwd, picks, picks_now  # the second workload reuses the first one's pinned pool block

    # The same forward loop with the speculative windowed prefetch (default budgets), on a
    # fresh copy of the workload so that both loops start from the same state.
    rot2, upd2, _ = synthetic.resident_workload(torch, kvip_amd, device, seed=seed, batch=batch, history=history,
                                                resident=resident, prefetch=kvip_amd.ResidentPrefetch())
    fwd2 = kvip_amd.LIFetch(rot2, upd2)
    upd2.attach_lru(kvip_amd.SlotLRUChains(torch, batch, resident, device, slots=upd2.lru_slots))
    q2 = rot2.query.view(torch.uint8)
    trace2 = torch.zeros((n, 2, batch), dtype=torch.int32, device=device)

    def prefetch_body(cursor):
        _pick(torch, queries, cursor, q2)
        fwd2()
        trace2.index_copy_(0, cursor, torch.stack([upd2.miss_counts[:, 4], upd2.prefetch_counts]).view(1, 2, batch))

    pf_us = _cursor_rounds(torch, prefetch_body, warm, rounds, n, label="resident prefetch forward")
    if upd2.status.any() or rot2.status.any():
        raise RuntimeError(f"resident prefetch forward failed: {upd2.status.cpu().tolist()}")
    pf_trace = trace2[warm:warm + rounds].sum(2).float().mean(0).tolist()
    out.update({"host_read_ceiling_gbs": round(host_read_gbs(torch, device), 1),
                "prefetch_forward_us": round(pf_us, 2), "prefetch_final_misses_per_round": round(pf_trace[0], 1),
                "prefetched_per_round": round(pf_trace[1], 1)})
    return out


def prefill_leg(torch, kvip_amd, device, seed, iters=5):
    """config 3: one 4096-row prefill chunk against a 65536-token context, right-
    down causal. Times, with HIP events on the launch stream, the MFMA scoring launch, the
    TopK-2048 launch and the Index update of the 4096 new rows (VllmIndexCacheStorage.
    ingest_prefill, one list launch after the first call imported the restored prefix).
    Scoring is priced against the dense fp8 MFMA peak with 2*64*128 flops per visible
    (query, key) pair. `index_update` is the device launch alone; `index_update_eager` the
    whole eager adapter step (host-built plan and its copies included)."""
    from types import SimpleNamespace as NS
    from kvip_amd import synthetic
    from kvip_amd.adapters.vllm.index_import import VllmIndexCacheStorage

    wl = synthetic.prefill_workload(torch, device, seed=seed)
    q_len, k_len, heads = wl["q_len"], wl["k_len"], wl["heads"]
    idx = kvip_amd.PrefillIndexer(torch, max_rows=q_len, max_context=k_len, max_sequences=1, device=device,
                                  heads=heads)
    idx.bind(wl["query"], wl["weights"], wl["query_scale"], wl["keys"], wl["key_scale"], wl["cu_seqlens_q"],
             wl["seq_lens_k"], wl["block_table"])
    storage = VllmIndexCacheStorage(torch, 1, k_len, 2048, device)
    plan = NS(owner=0, request="c3", start=k_len - q_len, begin=0, stop=q_len)
    storage.prepare([plan])
    cache = (wl["keys"].view(-1, 128, 1, 128), wl["key_scale"].view(-1, 128, 1))
    metadata = NS(block_size=128, block_table=wl["block_table"], slot_mapping=wl["slot_mapping"])

    def ingest():
        storage.ingest_prefill(cache, metadata, [plan], wl["positions"])

    stream = torch.cuda.current_stream()
    for _ in range(6):  # first launches (code-object loading, the prefix import, clocks) stay untimed
        idx.score()
        idx.select()
        ingest()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(iters)]
    for e in ev:
        e[0].record(stream)
        idx.score()
        e[1].record(stream)
        idx.select()
        e[2].record(stream)
        ingest()
        e[3].record(stream)
    torch.cuda.synchronize()
    if int(idx.status.item()) != 0 or int(storage.status.item()) != 0:
        raise RuntimeError("prefill leg: device status set")
    t = {name: float(np.mean([e[i].elapsed_time(e[i + 1]) for e in ev])) * 1e3
         for i, name in enumerate(["score", "topk", "index_update_eager"])}
    # The device part of the Index update: the step's one list launch (the 4096 rows'
    # sources and targets as ingest_prefill builds them), timed on its own; the eager step
    # above adds the host-built plan and its copies to the device.
    import ctypes
    from kvip_amd.runtime import abi
    tokens = torch.arange(plan.begin, plan.stop, device=device)
    sources = wl["slot_mapping"].to(torch.int64).index_select(0, tokens).contiguous()
    targets = (wl["positions"].to(torch.int64).index_select(0, tokens) + plan.owner * k_len).contiguous()
    pk, ps = cache[0].view(torch.uint8).reshape(-1, 128), cache[1].reshape(-1)
    iargs = abi.IngestArgs(source_keys=abi.ptr(pk), source_scales=abi.ptr(ps), target_keys=abi.ptr(storage.keys),
                           target_scales=abi.ptr(storage.scales), status=abi.ptr(storage.status),
                           source_rows=pk.shape[0], target_rows=storage.owners * storage.history,
                           mode=abi.INGEST_LIST, count=int(tokens.numel()), sources=abi.ptr(sources),
                           targets=abi.ptr(targets), target_base=0)
    lib = abi.load_library()
    torch.cuda.synchronize()
    uev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in uev:
        e0.record(stream)
        abi.check(lib.kvip_hip_ingest_index(ctypes.byref(iargs), stream.cuda_stream), "Index update")
        e1.record(stream)
    torch.cuda.synchronize()
    t["index_update"] = float(np.mean([e0.elapsed_time(e1) for e0, e1 in uev])) * 1e3
    vis = np.clip(k_len - q_len + np.arange(q_len) + 1, 0, k_len).astype(np.int64)
    pairs = int(vis.sum())
    flops = 2 * heads * 128 * pairs
    tflops = flops / (t["score"] * 1e-6) / 1e12
    topk_bytes = pairs * 2 + q_len * (256 * 4 * 2 + TOPK * 4)
    update_bytes = q_len * (2 * (128 + 4) + 2 * 8)
    total = t["score"] + t["topk"] + t["index_update"]

    # The same chunk with bf16 Q/K (no scales): scoring and TopK, priced against the dense
    # bf16 MFMA peak.
    wb = synthetic.prefill_workload(torch, device, seed=seed, qk="bf16")
    bidx = kvip_amd.PrefillIndexer(torch, max_rows=q_len, max_context=k_len, max_sequences=1, device=device,
                                   heads=heads)
    bidx.bind(wb["query"], wb["weights"], None, wb["keys"], None, wb["cu_seqlens_q"], wb["seq_lens_k"],
              wb["block_table"])
    for _ in range(3):
        bidx.score()
        bidx.select()
    torch.cuda.synchronize()
    bev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(iters)]
    for e in bev:
        e[0].record(stream)
        bidx.score()
        e[1].record(stream)
        bidx.select()
        e[2].record(stream)
    torch.cuda.synchronize()
    if int(bidx.status.item()) != 0:
        raise RuntimeError("prefill leg (bf16): device status set")
    bt = {name: float(np.mean([e[i].elapsed_time(e[i + 1]) for e in bev])) * 1e3
          for i, name in enumerate(["score", "topk"])}
    btflops = flops / (bt["score"] * 1e-6) / 1e12
    bf16 = {"us": {k: round(v, 1) for k, v in bt.items()},
            "score_roofline": {"bound": "mfma", "achieved": round(btflops, 1), "peak": BF16_MFMA_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(btflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops": flops}}
    return {"workload": f"c3: 1 sequence, {q_len} query rows x {k_len} context tokens, right-down causal, "
                        f"fp8 Q/K, {heads} heads x 128, per-token scales; TopK-2048 per row; Index update of "
                        f"{q_len} rows",
            "us": {k: round(v, 1) for k, v in t.items()}, "us_total": round(total, 1),
            "rows_per_s": round(q_len / (total * 1e-6), 1), "visible_pairs": pairs,
            "score_roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": FP8_MFMA_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(tflops / FP8_MFMA_PEAK_TFLOPS, 4),
                               "flops": flops},
            "topk_gbs": round(topk_bytes / (t["topk"] * 1e-6) / 1e9, 1),
            "index_update_gbs": round(update_bytes / (t["index_update"] * 1e-6) / 1e9, 1), "iters": iters,
            "bf16": bf16}


def sfa_leg(torch, kvip_amd, device, seed, iters=20):
    """The consumer of the selected rows: sparse attention of 64 decode rows over their
    2048 selected 656-byte KV rows (kvip_hip_sparse_attention), 16 heads (MLA heads per GPU
    at 8-way tensor parallelism) and 128 heads, on the gathered buffer of a contiguous Fetch
    (indices 0..2047) and on a resident hot cache (2048 random slots of 16384 per request).
    Each call is one launch; 10 calls are captured in a hipGraph and replayed."""
    from kvip_amd.operators.sfa import SparseAttention

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    rows, out = 64, {}
    for layout, per_row in (("gathered", TOPK), ("hot_cache", 16384)):
        blocks = rows * per_row // 128
        kv = torch.randint(0, 256, (blocks, 128, 656), generator=gen, device=device, dtype=torch.uint8) & 0x77
        # Finite rope features and key scales (as random bytes they would be arbitrary bf16 and
        # fp32 values, up to ~2^112, whose logits overflow fp32).
        rope = (torch.rand((blocks, 128, 64), generator=gen, device=device) * 2 - 1).to(torch.bfloat16)
        kv[:, :, 512:640] = rope.view(torch.uint8).view(blocks, 128, 128)
        scales = torch.rand((blocks, 128, 4), generator=gen, device=device) * 0.01 + 0.001
        kv[:, :, 640:656] = scales.view(torch.uint8).view(blocks, 128, 16)
        table = (torch.arange(rows, dtype=torch.int32, device=device)[:, None] * (per_row // 128) +
                 torch.arange(per_row // 128, dtype=torch.int32, device=device)[None, :]).contiguous()
        if per_row == TOPK:
            idx = torch.arange(TOPK, dtype=torch.int32, device=device).repeat(rows, 1)
        else:
            idx = torch.argsort(torch.rand((rows, per_row), generator=gen, device=device), dim=1)[:, :TOPK]
            idx = idx.to(torch.int32).contiguous()
        for heads in (16, 128):
            q = (torch.rand((rows, heads, 576), generator=gen, device=device) * 0.4 - 0.2).to(torch.bfloat16)
            op = SparseAttention(torch, rows=rows, heads=heads, device=device).bind(q, kv, table, idx)
            op()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(10):
                    op()
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            stream = torch.cuda.current_stream()
            e0.record(stream)
            for _ in range(iters):
                graph.replay()
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (iters * 10)
            if op.status.any():
                raise RuntimeError(f"sparse attention: device status {op.status.cpu().tolist()}")
            nbytes = rows * TOPK * (656 + 4) + rows * heads * (576 * 2 + 512 * 4)
            out[f"{layout}_h{heads}"] = {"us": round(us, 2), "bytes": nbytes,
                                         "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                                         "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    out["workload"] = ("sparse attention of 64 rows x 2048 selected 656-byte KV rows (bf16 query [heads, 576], "
                       "fp32 out [heads, 512]); bytes = KV rows + indices + query + output, each once")
    return out


def mixed_leg(torch, kvip_amd, device, seed, rounds=20, warm=4, sequential=False, prefill_after=None,
              prefill_workgroups=None):
    """config 5: continuous-batching rounds captured as hipGraphs (CURSOR_ROUNDS_PER_GRAPH
    rounds per graph), each round: Index ingest of all new tokens (32 decode + 2048 + 1536 prefill rows), resident decode
    LIFetch for 32 requests (ctx ~U[4096, 65536], 16384 hot slots, misses from pinned host
    memory, the LRU chains committed inside the graph) and prefill LI + TopK for the two
    chunks (k_len 8192 and 1536). Consecutive replays are consecutive serving rounds on the
    evolving cache state: each picks its decode queries by a device cursor from a random
    walk (overlapping, drifting selections) and records its misses. prefill_after: where
    the prefill stage forks off; prefill_workgroups: its scoring grid (MixedRound's defaults
    when None)."""
    from kvip_amd import synthetic

    wl = synthetic.mixed_workload(torch, kvip_amd, device, seed=seed, lru=True, overlap=not sequential,
                                  prefill_after=prefill_after, prefill_workgroups=prefill_workgroups)
    rnd = wl.round
    nd = len(wl.decode_ctx)
    n = warm + rounds + 1
    queries = _query_walk(torch, wl.rot.query, n, seed)
    q_bytes = wl.rot.query.view(torch.uint8)
    trace = torch.zeros((n, nd), dtype=torch.int32, device=device)

    def body(cursor):
        _pick(torch, queries, cursor, q_bytes)
        rnd()
        trace.index_copy_(0, cursor, wl.update.miss_counts[:, 4].view(1, nd))

    us = _cursor_rounds(torch, body, warm, rounds, n, label="mixed round")
    for st in (wl.update.status, wl.rot.status, wl.prefill.status, rnd.status):
        if st.any():
            raise RuntimeError(f"mixed round: device status {st.cpu().tolist()}")
    miss = trace[warm:warm + rounds].sum(1).float().mean().item()
    pf_rows = sum(q for q, _ in wl.chunks)
    return {"workload": f"c5: {nd} decode requests (ctx U[4096,{wl.history}], mean "
                        f"{wl.decode_ctx.mean():.0f}; resident {wl.resident} hot slots, misses from pinned host "
                        f"memory, LRU chains committed in the graph, queries along a random walk) + prefill "
                        f"chunks {[list(c) for c in wl.chunks]} (q_len, k_len); Index ingest of "
                        f"{len(wl.sources)} new tokens; each round one captured sequence, 4 rounds per hipGraph",
            "us_per_round": round(us, 1), "decode_rows": nd, "prefill_rows": pf_rows,
            "rows_per_s": round((nd + pf_rows) / (us * 1e-6), 1),
            "decode_misses_per_round": round(miss, 1),
            "decode_hit_fraction": round(1.0 - miss / (nd * TOPK), 4), "rounds": rounds,
            "rounds_per_graph": CURSOR_ROUNDS_PER_GRAPH,
            "prefill_workgroups": rnd.prefill_workgroups,
            "streams": "one" if sequential else (f"prefill forked after the decode's {rnd.prefill_after}"
                                                 if rnd.prefill_after != "start" else "prefill forked at the start")
                       + ("" if sequential else ", Fetch beside the Index update")}


def _stage_times(torch, pairs, per_graph=8, reps=25):
    """Per-stage device times of the three-launch round, in ms per round: graphs of
    `per_graph` back-to-back calls alternating over the `pairs` (LIFetch forwards of the two
    input sets), timed with HIP events on the launch stream. Scoring from score-only graphs,
    TopK as score+TopK minus scoring, the gather as the whole round minus score+TopK."""
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for f in pairs:
            f()
    stream.wait_stream(side)
    torch.cuda.synchronize()

    def graph_of(calls):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for j in range(per_graph):
                calls[j % 2]()
        return g

    def ms(g):
        for _ in range(3):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / (reps * per_graph)

    full = ms(graph_of(pairs))
    score = ms(graph_of([f.score for f in pairs]))
    for f in pairs:
        f.rotating.histogram.zero_()  # score-only replays keep adding to the histograms
    score_topk = ms(graph_of([lambda f=f: (f.score(), f.select()) for f in pairs]))
    return {"round": full, "indexer": score, "topk": score_topk - score, "fetch": full - score_topk}


def mtp_leg(torch, kvip_amd, device, seed):
    """The decode step as the vLLM selector runs it: 4 query rows per request (the MTP rows,
    python/kvip/adapters/vllm/inputs.py:11), at config-2 sizes (64 requests, ctx U[8192,
    32768], fp8, 64 heads, key scales, 656-byte KV rows). Row q of request b sees its first
    ctx_b - 3 + q tokens. Every index-K tile of a request is read once and scored for its 4
    rows, so a tile carries 4 x 2 x 64 x 128 flops per token against 132 bytes (496 flop/B
    against MI355X's fp8 ridge of 625 flop/B: HBM-bound, with the MFMA roof 1.26x away). Bytes
    count each index-K row once per request; the gather moves 4 x 2048 rows per request."""
    from kvip_amd import synthetic

    sets = []
    for k in range(2):
        wl = synthetic.decode_workload(torch, batch=64, ctx_low=8192, ctx_high=32768, device=device, qk="fp8",
                                       key_scale=True, rows_per_request=4, seed=seed + k, max_context=32768)
        ends = np.stack([wl.ctx - 3 + q for q in range(4)], axis=1).reshape(-1)
        sets.append((wl, *synthetic.bind(torch, kvip_amd, wl, query_ends=ends)))
    heads = int(sets[0][0].query.shape[1])
    per = [algorithmic_bytes(w, heads, False) for w, *_ in sets]
    mean = {k: (per[0][k] + per[1][k]) / 2 for k in per[0]}
    flops = float(np.mean([2 * heads * 128 * (np.minimum(w.ctx[:, None], np.stack([w.ctx - 3 + q for q in range(4)], 1))
                                             .sum()) for w, *_ in sets]))
    t = _stage_times(torch, [f for *_, f in sets])
    for w, r, u, f in sets:
        if int(r.status.item()) != 0:
            raise RuntimeError(f"MTP leg: device status {int(r.status.item())}")
    score_s = t["indexer"] * 1e-3
    hbm = mean["indexer"] / score_s / 1e9
    tflops = flops / score_s / 1e12
    step_bytes = sum(mean.values())
    rows = 64 * 4
    return {"workload": "c2 sizes with 4 MTP rows per request: 64 requests x 4 rows, ctx U[8192,32768], fp8, "
                        "64 heads x 128, key scales, KV rows 656 B, row q sees ctx - 3 + q tokens",
            "us_per_step": round(t["round"] * 1e3, 2), "queries_per_s": round(rows / (t["round"] * 1e-3), 1),
            "hbm_frac_step": round(step_bytes / (t["round"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernels_us": {k: round(v * 1e3, 2) for k, v in t.items() if k != "round"},
            "step_bytes": int(step_bytes), "score_flops": int(flops),
            "score_roofline": {"bound": "hbm", "achieved": round(hbm, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": round(hbm / HBM_PEAK_GBS, 4),
                               "mfma_tflops": round(tflops, 1), "mfma_frac": round(tflops / FP8_MFMA_PEAK_TFLOPS, 4)}}


def copy_calibration(torch, device):
    """Three plain 1 GiB device-to-device copies: the kernel whose rocprofv3 FETCH_SIZE and
    WRITE_SIZE per dispatch scale those counters to bytes moved."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the path shards by request with no "
              "exchange between GPUs). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import kvip_amd
    from kvip_amd import synthetic

    device = "cuda:0"
    torch.cuda.set_device(0)
    only_legs = {"mtp": lambda: mtp_leg(torch, kvip_amd, device, args.seed),
                 "lidu": lambda: lidu_leg(torch, kvip_amd, device, args.seed),
                 "resident": lambda: resident_leg(torch, kvip_amd, device, args.seed, sequential=args.sequential),
                 "cache_ops": lambda: cache_ops_leg(torch, kvip_amd, device, args.seed),
                 "prefill": lambda: prefill_leg(torch, kvip_amd, device, args.seed),
                 "mixed": lambda: mixed_leg(torch, kvip_amd, device, args.seed, sequential=args.sequential),
                 "sfa": lambda: sfa_leg(torch, kvip_amd, device, args.seed)}
    if args.only is not None:
        if args.only not in only_legs:
            raise SystemExit(f"--only: unknown leg {args.only!r} ({', '.join(only_legs)})")
        print(f"bench: {args.only} leg starts", file=sys.stderr, flush=True)
        print(json.dumps({"leg": args.only, args.only: only_legs[args.only]()}), flush=True)
        print(f"bench: {args.only} leg done", file=sys.stderr, flush=True)
        if args.copy_calibration:
            copy_calibration(torch, device)
        return
    # Two independent input sets, alternated step by step: a step touches ~346 MB and
    # MI355X's 256 MB Infinity Cache would otherwise keep part of the same inputs
    # between consecutive steps, so every step streams its inputs from HBM.
    sets = []
    for k in range(2):
        wl = synthetic.config_workload(torch, args.config, device, seed=args.seed + k)
        sets.append((wl, *synthetic.bind(torch, kvip_amd, wl)))
    wl, rot, upd, fwd = sets[0]
    heads = int(wl.query.shape[1])
    per_kernel_bytes = [algorithmic_bytes(w, heads, w.query_scale is not None) for w, *_ in sets]
    step_bytes = [sum(b.values()) for b in per_kernel_bytes]
    mean_bytes = {k: (per_kernel_bytes[0][k] + per_kernel_bytes[1][k]) / 2 for k in per_kernel_bytes[0]}

    for i in range(args.warmup):
        sets[i % 2][3]()
    torch.cuda.synchronize()
    for w, r, u, f in sets:
        if int(r.status.item()) != 0:
            raise RuntimeError(f"device status {int(r.status.item())} after warm-up")

    stream = torch.cuda.current_stream()
    # Timed region: `rounds_per_graph` decode rounds captured back to back in one hipGraph
    # (input sets alternating, kernel nodes with no host launch between them, as the
    # indexer runs inside a model's captured decode step), replayed until exactly
    # args.steps rounds have run; a remainder runs as one-round graphs. The forward is
    # graph-capturable: no allocation, sync or memset.
    per_graph = args.rounds_per_graph
    if per_graph < 1 or (per_graph > 1 and per_graph % 2):
        raise SystemExit("--rounds-per-graph must be 1 or even (the two input sets alternate)")
    graphs = []
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for w, r, u, f in sets:
            f()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    for w, r, u, f in sets:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f()
        graphs.append(g)
    multi = torch.cuda.CUDAGraph()
    with torch.cuda.graph(multi):
        for j in range(per_graph):
            sets[j % 2][3]()
    for i in range(4):
        graphs[i % 2].replay()
    multi.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps // per_graph):
        multi.replay()
    for s in range(args.steps - args.steps % per_graph, args.steps):
        graphs[s % 2].replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    steps_bytes = sum(step_bytes[s % 2] for s in range(args.steps))

    # Per-kernel durations: HIP events on the launch stream around replays of graphs of
    # `rounds_per_graph` back-to-back calls, same alternating inputs: scoring from
    # score-only graphs, TopK as score+TopK graphs minus scoring, the gather as the full
    # three-launch round minus score+TopK. graph_ms_per_step is the default round with one
    # graph launch per round.
    plan = fwd.plan
    threes = [kvip_amd.LIFetch(r, u) for w, r, u, f in sets]

    def capture(calls):
        gs = []
        for k in range(1 if per_graph > 1 else len(calls)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for j in range(per_graph):
                    calls[(k + j) % 2]()
            gs.append(g)
        return gs

    def replay_ms(gs):
        per = per_graph if len(gs) == 1 else 1
        reps = max(1, args.steps // per)
        for i in range(4):
            gs[i % len(gs)].replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for s in range(reps):
            gs[s % len(gs)].replay()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / (reps * per)

    with torch.cuda.stream(side):
        for t in threes:
            t()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    full_ms = replay_ms(graphs)
    score_ms = replay_ms(capture([t.score for t in threes]))
    for w, r, u, f in sets:
        r.histogram.zero_()  # score-only replays keep adding to the histograms
    st_ms = replay_ms(capture([lambda t=t: (t.score(), t.select()) for t in threes]))
    three_ms = replay_ms(capture(threes))
    times = {"indexer": score_ms, "topk": st_ms - score_ms, "fetch": three_ms - st_ms}
    for w, r, u, f in sets:
        if int(r.status.item()) != 0:
            raise RuntimeError(f"device status {int(r.status.item())} after the timed steps")

    if args.copy_calibration:
        copy_calibration(torch, device)

    rows = rot.rows
    # The dominant kernel of the default three-launch round: the longest launch.
    dominant = max(times, key=times.get)
    achieved = mean_bytes[dominant] / (times[dominant] * 1e-3) / 1e9
    result = {
        "metric": "decode queries/sec LI+TopK+Fetch, B=64 ctx 32k; achieved HBM GB/s vs peak",
        "value": round(rows * args.steps / wall, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if wl.query.element_size() == 1 else "bf16",
        "data": "synthetic (seeded N(0,1) fp8 Q/K, U(0.5,2) key scales, random KV bytes; two input sets alternated)",
        "config": {"workload": f"{args.config}: decode LI+TopK-2048+Fetch, batch {wl.batch}, "
                               f"ctx U[{int(wl.ctx.min())},{int(wl.ctx.max())}] (mean {wl.ctx.mean():.0f}), "
                               f"{heads} heads x 128, KV rows {int(wl.kv_cache.shape[2])} B",
                   "batch": wl.batch, "context_tokens": [int(w.ctx.sum()) for w, *_ in sets],
                   "seeds": [args.seed, args.seed + 1]},
        "hbm_gbs_step": round(steps_bytes / wall / 1e9, 1),
        "hbm_frac_step": round(steps_bytes / wall / 1e9 / HBM_PEAK_GBS, 4),
        "step_bytes": step_bytes,
        "plan": plan,
        "rounds_per_graph": per_graph,
        "graph_ms_per_step": round(full_ms, 4),
        "three_launch_graph_ms_per_step": round(three_ms, 4),
        "kernels": {k: {"ms": round(v, 5), "bytes": int(mean_bytes[k]),
                        "gbs": round(mean_bytes[k] / (v * 1e-3) / 1e9, 1)} for k, v in times.items()},
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(dominant) if args.config == "c2" else None},
    }
    legs = [("mtp", args.no_mtp, lambda: mtp_leg(torch, kvip_amd, device, args.seed)),
            ("lidu", args.no_lidu, lambda: lidu_leg(torch, kvip_amd, device, args.seed)),
            ("resident", args.no_resident, lambda: resident_leg(torch, kvip_amd, device, args.seed,
                                                                sequential=args.sequential)),
            ("cache_ops", args.no_resident, lambda: cache_ops_leg(torch, kvip_amd, device, args.seed)),
            ("prefill", args.no_prefill, lambda: prefill_leg(torch, kvip_amd, device, args.seed)),
            ("mixed", args.no_mixed, lambda: mixed_leg(torch, kvip_amd, device, args.seed,
                                                       sequential=args.sequential)),
            ("sfa", args.no_sfa, lambda: sfa_leg(torch, kvip_amd, device, args.seed)),
            ("cpu_baseline", args.no_cpu_baseline, lambda: cpu_baseline(torch, wl, rot, args.cpu_seconds))]
    print(f"bench: decode steps done ({result['ms_per_step']} ms/step)", file=sys.stderr, flush=True)
    for name, skip, leg in legs:
        if not skip:
            result[name] = leg()
            print(f"bench: {name} leg done", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
