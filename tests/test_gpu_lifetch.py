"""GPU parity of the decode LIFetch path (scoring -> TopK-2048 -> Fetch gather) against
the CPU oracle, through the C ABI of libkvip_hip.so.

Bars (written in each test): scores within 3e-2 relative for fp8 and 1e-2 for bf16
(with an absolute floor of the same fraction of the row's largest |score|, for
scores that cancel to near zero) and over 99 % of the keys with |score| >= 3e-2 of the
row's largest bit-identical; TopK bit-exact, order included, when fed the
oracle's keys; gather byte-exact."""
import ctypes

import numpy as np
import pytest

import kvip_amd
from kvip_amd import synthetic
from kvip_amd.runtime import abi
from oracle import indexer as ref

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)


def host_values(torch, t):
    if t is None:
        return None
    if t.dtype == torch.float8_e4m3fn:
        return ref.fp8_e4m3_decode(t.view(torch.uint8).cpu().numpy())
    return t.float().cpu().numpy()


def oracle_keys(torch, wl, rot):
    return ref.decode_keys_paged(
        host_values(torch, wl.query), host_values(torch, wl.weights), host_values(torch, wl.query_scale),
        host_values(torch, wl.keys), host_values(torch, wl.key_scale), wl.block_table.cpu().numpy(), wl.ctx,
        rows_per_request=wl.rows_per_request,
        query_ends=None if rot.query_ends is None else rot.query_ends.cpu().numpy(), key_stride=rot.key_stride)


def gpu_keys(rot):
    return rot.score_keys.cpu().numpy().view(np.uint16)


def assert_scores_close(got_keys, want_keys, valid, rtol):
    for r, v in enumerate(valid):
        if v == 0:
            continue
        g = ref.score_values(got_keys[r, :v]).astype(np.float64)
        w = ref.score_values(want_keys[r, :v]).astype(np.float64)
        floor = rtol * np.abs(w).max()
        bad = np.abs(g - w) > rtol * np.abs(w) + floor
        assert not bad.any(), f"row {r}: {bad.sum()} scores outside rtol {rtol}"
    same = ref.identical_share(got_keys, want_keys, valid)
    say(f"  identical keys (|score| >= 3e-2 of row max): {same:.5f}")
    assert same > 0.99


CASES = [
    # name, qk, heads, weight dtype, key scale, query scale, ctx
    ("fp8_h64_fp32w", "fp8", 64, "f32", True, True, [1, 100, 2047, 2048, 5000, 9000]),
    ("fp8_h32_bf16w", "fp8", 32, "bf16", True, False, [4096, 3000, 129]),
    ("bf16_h64_c1", "bf16", 64, "f32", False, False, [4096, 4096, 4096, 4096]),
]


@pytest.mark.parametrize("name,qk,heads,wdt,kscale,qscale,ctx", CASES, ids=[c[0] for c in CASES])
def test_indexer_scores_match_oracle(torch_gpu, name, qk, heads, wdt, kscale, qscale, ctx):
    torch = torch_gpu
    say(f"case {name}")
    wl = synthetic.decode_workload(torch, batch=len(ctx), ctx=ctx, device="cuda", heads=heads, qk=qk,
                                   weight_dtype=torch.float32 if wdt == "f32" else torch.bfloat16,
                                   key_scale=kscale, query_scale=qscale, seed=11)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd.score()
    torch.cuda.synchronize()
    want, valid = oracle_keys(torch, wl, rot)
    assert_scores_close(gpu_keys(rot), want, valid, 3e-2 if qk == "fp8" else 1e-2)
    assert int(rot.status.item()) == 0
    # Histogram of high bytes over the valid prefix equals the keys' own histogram.
    hist = rot.histogram.cpu().numpy()
    for r, v in enumerate(valid):
        assert np.array_equal(hist[r], np.bincount(gpu_keys(rot)[r, :v] >> 8, minlength=256)), r


MTP_CASES = [
    # name, rows per request, heads, weight dtype, key scale, query scale, ctx
    ("rows4_h64_fp32w", 4, 64, "f32", True, True, [9000, 4100, 33, 12000, 1, 2049]),
    ("rows2_h64_bf16w", 2, 64, "bf16", True, False, [5000, 31, 7000]),
    ("rows4_h32_noscale", 4, 32, "f32", False, False, [3000, 4096, 130]),
]


@pytest.mark.parametrize("name,rows,heads,wdt,kscale,qscale,ctx", MTP_CASES, ids=[c[0] for c in MTP_CASES])
def test_indexer_mtp_rows_match_oracle(torch_gpu, name, rows, heads, wdt, kscale, qscale, ctx):
    """fp8 decode scoring with 2 or 4 query rows per request (the shared-ring kernel): row q
    of request b sees its own visible bound (ctx - rows + 1 + q, with a padding row and rows
    shorter than one tile); keys against the oracle and every row's histogram against its
    keys."""
    torch = torch_gpu
    say(f"case {name}")
    wl = synthetic.decode_workload(torch, batch=len(ctx), ctx=ctx, device="cuda", heads=heads, qk="fp8",
                                   weight_dtype=torch.float32 if wdt == "f32" else torch.bfloat16,
                                   key_scale=kscale, query_scale=qscale, rows_per_request=rows, seed=13)
    ends = []
    for c in ctx:
        ends += [max(c - rows + 1 + q, 0) for q in range(rows)]
    ends[1] = 0  # a padding row
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl, query_ends=ends)
    fwd.score()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    want, valid = oracle_keys(torch, wl, rot)
    assert list(valid) == [min(e, c) for e, c in zip(ends, np.repeat(ctx, rows))]
    assert_scores_close(gpu_keys(rot), want, valid, 3e-2)
    hist = rot.histogram.cpu().numpy()
    for r, v in enumerate(valid):
        assert np.array_equal(hist[r], np.bincount(gpu_keys(rot)[r, :v] >> 8, minlength=256)), r


def run_topk(torch, rot, use_histogram, split=True):
    lib = abi.load_library()
    args = rot.topk_args(use_histogram, split=split)
    rc = lib.kvip_hip_topk(ctypes.byref(args), abi.stream_handle(torch, rot.device))
    abi.check(rc, "topk")
    torch.cuda.synchronize()
    return rot.topk.cpu().numpy()


def keys_case(kind, n, rng):
    if kind == "random":
        return ref.sortable_key(ref.bf16_round_half_away(rng.standard_normal(n).astype(np.float32) * 8))
    if kind == "few_levels":
        return (0x8000 + rng.integers(0, 5, n)).astype(np.uint16)
    if kind == "all_equal":
        return np.full(n, 0xC200, np.uint16)
    if kind == "one_bin":
        return (0xC200 + rng.integers(0, 256, n)).astype(np.uint16)
    raise ValueError(kind)


@pytest.mark.parametrize("kind,ctx", [
    ("random", [32768, 20000, 2048, 2047, 0, 8193]),
    ("random", [8192, 5000, 2049, 100]),  # rows of at most 8192 keys: 256-thread workgroups
    ("few_levels", [16384, 30000]),
    ("all_equal", [4096, 2048]),
    ("all_equal", [65536, 4096]),  # a full register row of equal keys: the eq total reaches 65536
    ("one_bin", [131072]),
])
def test_topk_bit_exact_on_oracle_keys(torch_gpu, kind, ctx):
    torch = torch_gpu
    say(f"case topk {kind} {ctx}")
    rng = np.random.default_rng(len(ctx) * 7 + ctx[0])
    rot = kvip_amd.LIFetchBinding(torch, batch=len(ctx), max_context=max(max(ctx), 1), device="cuda")
    keys = np.zeros((len(ctx), rot.key_stride), np.uint16)
    for r, v in enumerate(ctx):
        keys[r, :v] = keys_case(kind, v, rng)
    rot.score_keys.copy_(torch.from_numpy(keys.view(np.int16)))
    rot.seq_lens.copy_(torch.tensor(ctx, dtype=torch.int32))
    got = run_topk(torch, rot, use_histogram=False)
    for r, v in enumerate(ctx):
        want = ref.topk_reference(keys[r], v)
        assert np.array_equal(got[r], want), f"row {r} valid {v}"
    assert int(rot.status.item()) == 0
    # The multi-workgroup select, fed the rows' high-byte histogram as the scoring kernel
    # leaves it, gives the same rows and clears the histogram.
    hist = np.stack([np.bincount(keys[r, :v] >> 8, minlength=256) for r, v in enumerate(ctx)])
    rot.histogram.copy_(torch.from_numpy(hist.astype(np.int32)))
    rot.topk.fill_(-5)
    say(f"case topk split {kind} {ctx}")
    got = run_topk(torch, rot, use_histogram=True)
    for r, v in enumerate(ctx):
        assert np.array_equal(got[r], ref.topk_reference(keys[r], v)), f"split row {r} valid {v}"
    assert int(rot.status.item()) == 0
    assert not rot.histogram.any()
    # The forward's select: keys in registers, the high-byte bin from the same histogram.
    rot.histogram.copy_(torch.from_numpy(hist.astype(np.int32)))
    rot.topk.fill_(-5)
    say(f"case topk registers+histogram {kind} {ctx}")
    got = run_topk(torch, rot, use_histogram=True, split=False)
    for r, v in enumerate(ctx):
        assert np.array_equal(got[r], ref.topk_reference(keys[r], v)), f"register row {r} valid {v}"
    assert int(rot.status.item()) == 0
    assert not rot.histogram.any()


def test_topk_reports_a_histogram_that_misses_keys(torch_gpu):
    """A scoring histogram whose total differs from the row's visible keys (a skipped or
    repeated tile) is reported in the status word instead of passing silently."""
    torch = torch_gpu
    rng = np.random.default_rng(17)
    rot = kvip_amd.LIFetchBinding(torch, batch=1, max_context=8192, device="cuda")
    keys = np.zeros((1, rot.key_stride), np.uint16)
    keys[0, :8192] = keys_case("random", 8192, rng)
    rot.score_keys.copy_(torch.from_numpy(keys.view(np.int16)))
    rot.seq_lens.copy_(torch.tensor([8192], dtype=torch.int32))
    hist = np.bincount(keys[0, :8192] >> 8, minlength=256)
    hist[int(np.argmax(hist))] -= 32  # one 32-token tile missing from the counts
    rot.histogram.copy_(torch.from_numpy(hist[None, :].astype(np.int32)))
    run_topk(torch, rot, use_histogram=True, split=False)
    assert int(rot.status.item()) & abi.STATUS_HISTOGRAM


def test_topk_from_scoring_histogram_equals_standalone(torch_gpu):
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=5, ctx=[9000, 2048, 100, 17000, 4097], device="cuda", seed=3)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd.score()
    fwd.select()
    torch.cuda.synchronize()
    fused = rot.topk.cpu().numpy().copy()
    assert not rot.histogram.cpu().numpy().any(), "TopK must re-zero the histogram"
    alone = run_topk(torch, rot, use_histogram=False)
    assert np.array_equal(fused, alone)
    keys = gpu_keys(rot)
    for r, v in enumerate(wl.ctx):
        assert np.array_equal(fused[r], ref.topk_reference(keys[r], v))


def test_fetch_gather_byte_exact(torch_gpu):
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=4, ctx=[3000, 1000, 6000, 2048], device="cuda", seed=5)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd()
    torch.cuda.synchronize()
    topk = rot.topk.cpu().numpy()
    want = ref.fetch_gather(wl.kv_cache.cpu().numpy(), wl.block_table.cpu().numpy(), topk)
    assert np.array_equal(upd.output.cpu().numpy(), want)
    assert (topk[1, 1000:] == -1).all() and not upd.output[1, 1000:].any()
    assert int(rot.status.item()) == 0


def test_forward_end_to_end_against_oracle_scores(torch_gpu):
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=8, ctx_low=8192, ctx_high=20000, device="cuda", seed=2026)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd()
    torch.cuda.synchronize()
    want, valid = oracle_keys(torch, wl, rot)
    topk = rot.topk.cpu().numpy()
    for r, v in enumerate(valid):
        assert ref.validate_topk_band(topk[r], ref.score_values(want[r, :v])), r
        # Bit-exact against the oracle's TopK of the GPU's own keys.
        assert np.array_equal(topk[r], ref.topk_reference(gpu_keys(rot)[r], v))
    out = upd.output.cpu().numpy()
    assert np.array_equal(out, ref.fetch_gather(wl.kv_cache.cpu().numpy(), wl.block_table.cpu().numpy(), topk))


def test_forward_deferred_fetch_option_changes_nothing(torch_gpu):
    """set_options(deferred_fetch=True), the reference harness's set_deferred_fetch, leaves
    the round's TopK and gathered rows byte-identical to the default forward's."""
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=4, ctx_low=4096, ctx_high=12000, device="cuda", seed=77)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    results = []
    for deferred in (False, True, False):
        say(f"forward deferred_fetch={deferred}")
        fwd.set_options(deferred_fetch=deferred)
        rot.topk.fill_(-5)
        upd.output.fill_(0xAB)
        fwd()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        results.append((rot.topk.cpu().numpy(), upd.output.cpu().numpy()))
    for topk, out in results[1:]:
        assert np.array_equal(topk, results[0][0]) and np.array_equal(out, results[0][1])


def test_forward_mtp_rows_against_oracle(torch_gpu):
    """Four query rows per request (decode + 3 MTP rows) with per-row visible bounds: the
    forward's scores, TopK (bit-exact on the GPU's keys, inside the oracle's cutoff band) and
    gather."""
    torch = torch_gpu
    ctx = [9000, 4100, 2200, 12000]
    wl = synthetic.decode_workload(torch, batch=4, ctx=ctx, device="cuda", rows_per_request=4, seed=44)
    ends = []
    for c in ctx:
        ends += [c - 3, c - 2, c - 1, c]
    ends[6] = 0          # a padding row
    ends[9] = 2047       # a row below 2048 visible tokens
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl, query_ends=ends)
    assert fwd.plan == "three"
    fwd()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    want, valid = oracle_keys(torch, wl, rot)
    keys = gpu_keys(rot)
    assert_scores_close(keys, want, valid, 3e-2)
    topk = rot.topk.cpu().numpy()
    for r, v in enumerate(valid):
        assert np.array_equal(topk[r], ref.topk_reference(keys[r], v)), r
        if v >= 2048:
            assert ref.validate_topk_band(topk[r], ref.score_values(want[r, :v])), r
    assert (topk[6] == -1).all()
    assert np.array_equal(topk[9, :2047], np.arange(2047)) and topk[9, 2047] == -1
    table = wl.block_table.cpu().numpy()
    assert np.array_equal(upd.output.cpu().numpy(), ref.fetch_gather(wl.kv_cache.cpu().numpy(), table, topk,
                                                                     rows_per_request=4))


def test_graph_replay_matches_eager(torch_gpu):
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=6, ctx_low=3000, ctx_high=12000, device="cuda", seed=9)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fwd()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    gen = torch.Generator(device="cuda")
    for step in range(3):
        gen.manual_seed(100 + step)
        new_q = synthetic.saturating_fp8(torch, torch.randn(rot.query.shape, generator=gen, device="cuda"))
        rot.query.copy_(new_q)
        graph.replay()
        torch.cuda.synchronize()
        g_topk, g_out = rot.topk.clone(), upd.output.clone()
        rot.topk.fill_(-7)
        fwd()
        torch.cuda.synchronize()
        assert torch.equal(g_topk, rot.topk), step
        assert torch.equal(g_out, upd.output), step


def test_graph_of_alternating_rounds_matches_eager(torch_gpu):
    """Four decode rounds captured in one graph over two bound input sets (set 0, 1, 0, 1),
    the way bench.py times the step: every replay leaves each set's TopK and gathered rows
    equal to an eager round on that set."""
    torch = torch_gpu
    bound = [synthetic.bind(torch, kvip_amd, synthetic.decode_workload(
        torch, batch=6, ctx_low=3000, ctx_high=12000, device="cuda", seed=seed)) for seed in (11, 12)]
    want = []
    for rot, upd, fwd in bound:
        fwd()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        want.append((rot.topk.clone(), upd.output.clone()))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _, _, fwd in bound:
            fwd()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for j in range(4):
            bound[j % 2][2]()
    for rep in range(3):
        for rot, upd, _ in bound:
            rot.topk.fill_(-7)
            upd.output.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, ((rot, upd, _), (topk, out)) in enumerate(zip(bound, want)):
            assert int(rot.status.item()) == 0, (rep, k)
            assert torch.equal(rot.topk, topk), (rep, k)
            assert torch.equal(upd.output, out), (rep, k)


def test_bad_block_id_is_reported_not_faulted(torch_gpu):
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=2, ctx=[4096, 4096], device="cuda", seed=1)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    rot.block_table[1, 3] = rot.num_blocks + 5  # out of range: kernels skip the access
    fwd()
    torch.cuda.synchronize()
    assert int(rot.status.item()) & abi.STATUS_BAD_BLOCK


@pytest.mark.parametrize("kind,ctx", [
    ("random", [32768, 20000, 2048, 2047, 0, 8193, 2049]),
    ("few_levels", [16384, 30000, 4096]),
    ("all_equal", [6144, 2048]),
    ("one_bin", [32768, 2100]),
])
def test_select_fetch_matches_topk_then_gather(torch_gpu, kind, ctx):
    """The fused TopK+Fetch launch, fed oracle keys and their high-byte histogram, gives
    the oracle's TopK (bit-exact, order included) and its byte-exact gather; run twice
    in a row so the second launch starts from the counters the first one left."""
    torch = torch_gpu
    rng = np.random.default_rng(len(ctx) * 13 + ctx[0])
    rot = kvip_amd.LIFetchBinding(torch, batch=len(ctx), max_context=max(ctx), device="cuda")
    blocks = rot.batch * rot.max_blocks
    table = rng.permutation(blocks).astype(np.int32).reshape(rot.batch, rot.max_blocks)
    kv = rng.integers(0, 256, (blocks, 128, 656), dtype=np.uint8)
    kv_dev = torch.from_numpy(kv).to("cuda")
    rot.block_table.copy_(torch.from_numpy(table))
    rot.bind_index_cache(torch.zeros((blocks, 128, 128), dtype=torch.float8_e4m3fn, device="cuda"))
    upd = kvip_amd.ContiguousFetch(torch, rot, kv_dev)
    fwd = kvip_amd.LIFetch(rot, upd)
    keys = np.zeros((len(ctx), rot.key_stride), np.uint16)
    for r, v in enumerate(ctx):
        keys[r, :v] = keys_case(kind, v, rng)
    hist = np.stack([np.bincount(keys[r, :v] >> 8, minlength=256) for r, v in enumerate(ctx)])
    rot.score_keys.copy_(torch.from_numpy(keys.view(np.int16)))
    rot.seq_lens.copy_(torch.tensor(ctx, dtype=torch.int32))
    want_topk = np.stack([ref.topk_reference(keys[r], v) for r, v in enumerate(ctx)])
    want_rows = ref.fetch_gather(kv, table, want_topk)
    for attempt in range(2):
        say(f"case select_fetch {kind} {ctx} attempt {attempt}")
        rot.histogram.copy_(torch.from_numpy(hist.astype(np.int32)))
        rot.topk.fill_(-5)
        upd.output.fill_(0xAB)
        fwd.select_fetch()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        assert np.array_equal(rot.topk.cpu().numpy(), want_topk), attempt
        assert np.array_equal(upd.output.cpu().numpy(), want_rows), attempt
        assert not rot.histogram.any()
        # Every arrival counter is back at zero.
        assert not rot.topk_segments[:, 0, -1].any()


def test_select_fetch_rejects_rows_beyond_32768_and_forward_falls_back(torch_gpu):
    """Rows longer than 32768 keys are outside the fused launch (arguments rejected before
    anything runs); the forward, which runs TopK and Fetch as separate launches, takes them."""
    torch = torch_gpu
    wl = synthetic.decode_workload(torch, batch=2, ctx=[40000, 5000], device="cuda", seed=4)
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    with pytest.raises(ValueError):
        fwd.select_fetch()
    fwd()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    topk = rot.topk.cpu().numpy()
    keys = gpu_keys(rot)
    for r, v in enumerate(wl.ctx):
        assert np.array_equal(topk[r], ref.topk_reference(keys[r], v))
    assert np.array_equal(upd.output.cpu().numpy(),
                          ref.fetch_gather(wl.kv_cache.cpu().numpy(), wl.block_table.cpu().numpy(), topk))
