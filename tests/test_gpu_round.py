"""GPU parity of the XCD-local decode round (score_select.hip: scoring with each request
selected by the workgroup that finishes it, then the checked gather; through
kvip_hip_lifetch_forward with the round work memory) against the default three-launch
round (scoring, TopK, gather) on the same inputs.

Bars: TopK ids and every gathered byte bit-exact; the device status clear; the work memory
left zero after every launch (two eager launches in a row and graph replays agree); the
scores of rows of at least 2048 tokens bit-identical to the scoring kernel's."""
import numpy as np
import pytest

import kvip_amd
from kvip_amd import synthetic

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)


CASES = [
    # name, ctx, heads, weight dtype, key scale, query scale, query ends
    ("h64_mixed_lengths", [32768, 20000, 2048, 2047, 0, 8193, 2049, 100, 30000, 12345], 64, "f32", True, False, None),
    ("h64_qscale_bf16w", [9000, 4096, 17000, 2500], 64, "bf16", True, True, None),
    ("h32_no_kscale", [6000, 2048, 15000], 32, "f32", False, True, None),
    ("h64_query_ends", [20000, 9000, 5000, 3000], 64, "f32", True, False, [19990, 2047, 5000, 2600]),
]


def pair(torch, ctx, heads, wdt, kscale, qscale, ends, seed):
    wl = synthetic.decode_workload(torch, batch=len(ctx), ctx=ctx, device="cuda", heads=heads, qk="fp8",
                                   weight_dtype=torch.float32 if wdt == "f32" else torch.bfloat16,
                                   key_scale=kscale, query_scale=qscale, seed=seed, max_context=32768)
    rot, upd, _ = synthetic.bind(torch, kvip_amd, wl, query_ends=ends)
    fused = kvip_amd.LIFetch(rot, upd, fused=True)
    two = kvip_amd.LIFetch(rot, upd, fused=False)
    assert fused.plan == "round" and two.plan == "three"
    return wl, rot, upd, fused, two


@pytest.mark.parametrize("name,ctx,heads,wdt,kscale,qscale,ends", CASES, ids=[c[0] for c in CASES])
def test_round_matches_two_launch_round(torch_gpu, name, ctx, heads, wdt, kscale, qscale, ends):
    torch = torch_gpu
    say(f"case round {name}")
    wl, rot, upd, fused, two = pair(torch, ctx, heads, wdt, kscale, qscale, ends, seed=31)
    two()
    torch.cuda.synchronize()
    assert int(rot.status.item()) == 0
    want_topk, want_out = rot.topk.clone(), upd.output.clone()
    want_keys = rot.score_keys.clone()
    for launch in range(2):
        rot.topk.fill_(-7)
        upd.output.fill_(0x5A)
        rot.score_keys.zero_()
        fused()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0, launch
        assert torch.equal(rot.topk, want_topk), launch
        assert torch.equal(upd.output, want_out), launch
        assert not rot.round_work.any(), launch  # the work memory is left zero
        for r in range(rot.rows):
            v = min(ctx[r], ends[r]) if ends is not None else ctx[r]
            if v >= 2048:
                assert torch.equal(rot.score_keys[r, :v], want_keys[r, :v]), (launch, r)


def test_round_graph_replay(torch_gpu):
    torch = torch_gpu
    ctx = [32768, 20000, 2048, 2047, 0, 8193, 2049, 26000]
    say("case round graph replay")
    wl, rot, upd, fused, two = pair(torch, ctx, 64, "f32", True, False, None, seed=8)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fused()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fused()
    gen = torch.Generator(device="cuda")
    for step in range(3):
        gen.manual_seed(200 + step)
        rot.query.copy_(synthetic.saturating_fp8(torch, torch.randn(rot.query.shape, generator=gen, device="cuda")))
        graph.replay()
        torch.cuda.synchronize()
        g_topk, g_out = rot.topk.clone(), upd.output.clone()
        two()
        torch.cuda.synchronize()
        assert torch.equal(g_topk, rot.topk), step
        assert torch.equal(g_out, upd.output), step
        assert int(rot.status.item()) == 0, step


def test_round_config2_shape(torch_gpu):
    """BASELINE config 2 (64 requests, ctx U[8192, 32768], fp8, key scales): the round plan
    against the two-launch plan, both input seeds of the benchmark."""
    torch = torch_gpu
    for seed in (2026, 2027):
        say(f"case round config2 seed {seed}")
        wl = synthetic.config_workload(torch, "c2", "cuda", seed=seed)
        rot, upd, _ = synthetic.bind(torch, kvip_amd, wl)
        fused = kvip_amd.LIFetch(rot, upd, fused=True)
        two = kvip_amd.LIFetch(rot, upd, fused=False)
        assert fused.plan == "round"
        two()
        torch.cuda.synchronize()
        want_topk, want_out = rot.topk.clone(), upd.output.clone()
        for launch in range(2):
            rot.topk.fill_(-7)
            upd.output.fill_(0x5A)
            fused()
            torch.cuda.synchronize()
            assert int(rot.status.item()) == 0, launch
            assert torch.equal(rot.topk, want_topk), launch
            assert torch.equal(upd.output, want_out), launch
            assert not rot.round_work.any(), launch
            assert not rot.histogram.any(), launch
