"""GPU parity of the mixed continuous-batching round (kvip.MixedRound, config 5
shape at test size): Index ingest of the round's new tokens, resident decode LIFetch and
prefill LI + TopK, captured as one hipGraph.

Bars: a replay equals the same round run eagerly from the same state (every output, status
and Index/slot table bit-exact); the ingest copies every new token's index-K row and scale
bit-exactly; prefill scores within 3e-2 (fp8) and TopK bit-exact on the GPU keys; decode TopK
bit-exact on the GPU keys and inside the oracle's one-ulp cutoff band."""
import numpy as np
import pytest

import kvip_amd
from kvip_amd import synthetic
from oracle import indexer as ref

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)


def host(torch, t):
    if t.dtype == torch.float8_e4m3fn:
        return ref.fp8_e4m3_decode(t.view(torch.uint8).cpu().numpy())
    return t.float().cpu().numpy()


def small(torch, prefill_after=None):
    return synthetic.mixed_workload(torch, kvip_amd, "cuda", seed=7, decode_ctx=[8000, 5000, 6200, 3000],
                                    history=8192, resident=4096, prefill=((40, 3000), (25, 25)),
                                    prefill_after=prefill_after)


def state(wl):
    return [wl.keys, wl.scales, wl.addresses, wl.logical, wl.valid, wl.hot]


def outputs(wl):
    return [wl.update.outputs, wl.update.miss_counts, wl.update.status, wl.rot.topk, wl.rot.status,
            wl.prefill.topk, wl.prefill.row_valid, wl.prefill.status, wl.round.status]


def test_mixed_round_ingest_is_byte_exact(torch_gpu):
    torch = torch_gpu
    wl = small(torch)
    say("case mixed ingest")
    wl.round.ingest()
    torch.cuda.synchronize()
    assert int(wl.round.status.item()) == 0
    src_k = wl.cache_keys.view(torch.uint8).view(-1, 128).cpu().numpy()
    src_s = wl.cache_scales.view(-1).cpu().numpy()
    dst_k = wl.keys.view(torch.uint8).view(-1, 128).cpu().numpy()
    dst_s = wl.scales.view(-1).cpu().numpy()
    s = np.asarray(wl.sources)
    t = np.asarray(wl.targets)
    assert np.array_equal(dst_k[t], src_k[s])
    assert np.array_equal(dst_s[t], src_s[s])


@pytest.mark.parametrize("prefill_after", ["resolve", "scoring", "start"])
def test_mixed_round_graph_replay_matches_eager_and_oracle(torch_gpu, prefill_after):
    torch = torch_gpu
    wl = small(torch, prefill_after)
    assert wl.round.prefill_after == prefill_after
    start = [x.clone() for x in state(wl)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        wl.round()  # first launches outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        wl.round()
    for step in range(2):
        say(f"case mixed graph replay step {step} (prefill after {prefill_after})")
        for x, s in zip(state(wl), start):
            x.copy_(s)
        graph.replay()
        torch.cuda.synchronize()
        got = [x.clone() for x in state(wl) + outputs(wl)]
        for x, s in zip(state(wl), start):
            x.copy_(s)
        for o in (wl.update.outputs, wl.rot.topk, wl.prefill.topk):
            o.fill_(-9)
        wl.round()
        torch.cuda.synchronize()
        for i, (g, w) in enumerate(zip(got, state(wl) + outputs(wl))):
            assert torch.equal(g, w), (step, i)
    for s in (wl.update.status, wl.rot.status, wl.prefill.status, wl.round.status):
        assert not s.any()

    # Prefill rows against the oracle on the paged cache.
    p = wl.prefill
    want, vis = ref.prefill_keys_paged(host(torch, wl.pf_query), wl.pf_weights.cpu().numpy(),
                                       wl.pf_qscale.cpu().numpy(), host(torch, wl.cache_keys),
                                       wl.cache_scales.cpu().numpy(), wl.table.cpu().numpy(), wl.cu.cpu().numpy(),
                                       wl.kl.cpu().numpy(), p.key_stride)
    rows = len(vis)
    assert np.array_equal(p.row_valid[:rows].cpu().numpy(), vis)
    got = p.score_keys[:rows].cpu().numpy().view(np.uint16)
    for r, v in enumerate(vis):
        g = ref.score_values(got[r, :v]).astype(np.float64)
        w = ref.score_values(want[r, :v]).astype(np.float64)
        assert not (np.abs(g - w) > 3e-2 * np.abs(w) + 3e-2 * np.abs(w).max()).any(), r
    assert ref.identical_share(got, want, vis) > 0.99
    top = p.topk[:rows].cpu().numpy()
    for r, v in enumerate(vis):
        assert np.array_equal(top[r], ref.topk_reference(got[r], v)), r

    # Decode rows: scores over the owners' Index rows after the ingest.
    for x, s in zip(state(wl), start):
        x.copy_(s)
    wl.round.ingest()
    torch.cuda.synchronize()
    keys = host(torch, wl.keys)
    scales = wl.scales.cpu().numpy()
    q = host(torch, wl.rot.query)
    w = wl.rot.weights.float().cpu().numpy()
    qs = wl.rot.query_scale.cpu().numpy()
    gpu = got_dec = wl.rot.score_keys.cpu().numpy().view(np.uint16)
    dec_top = wl.rot.topk.cpu().numpy()
    for b, ctx in enumerate(wl.decode_ctx):
        ctx = int(ctx)
        want_b = ref.li_keys(q[b], keys[b, :ctx], w[b], qs[b], scales[b, :ctx])
        g = ref.score_values(got_dec[b, :ctx]).astype(np.float64)
        ww = ref.score_values(want_b).astype(np.float64)
        assert not (np.abs(g - ww) > 3e-2 * np.abs(ww) + 3e-2 * np.abs(ww).max()).any(), b
        assert np.array_equal(dec_top[b], ref.topk_reference(gpu[b], ctx)), b
        assert ref.validate_topk_band(dec_top[b], ref.score_values(want_b)), b
