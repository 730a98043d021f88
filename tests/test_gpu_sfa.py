"""GPU parity of the sparse-attention consumer (kvip_hip_sparse_attention through
kvip_amd.sparse_attention) against oracle/sfa.py, on the reference's KV payload rows.

Bars: the reference's own tolerance for this check (allclose atol 0.006, rtol 0.025,
correctness.py:329-330) and, tighter, a maximum absolute error below 3e-3; rows with no
valid index give zeros; bad positions are reported in status. Three sources of rows: a paged
cache with random indices (8, 16, 24, 40, 72 and 128 heads: one head group per workgroup, two
groups sharing each staged tile (24: the second group partly filled), a set whose second group
holds no heads; absent and repeated
indices; and, with enough rows that no index split is needed, 256 rows at 16 heads and 128
rows at 128 heads, whose workgroups write the normalised output themselves), the gathered
buffer of the contiguous LIFetch forward, and the resident hot cache addressed by the slot
outputs (the reference's check_sfa flow: slots from the round, values from the logical
tokens' payload)."""
import numpy as np
import pytest

import kvip_amd
from kvip_amd import synthetic
from kvip_amd.operators.sfa import gathered_table, hot_cache_table, sparse_attention
from oracle import sfa

pytestmark = pytest.mark.gpu
TOPK = 2048
ROW = 656
SCALE = 576 ** -0.5


def say(*args):
    print(*args, flush=True)


def bf16_query(torch, rng, rows, heads):
    q = rng.uniform(-0.2, 0.2, (rows, heads, 576)).astype(np.float32)
    qt = torch.from_numpy(q).to(torch.bfloat16)
    return qt.cuda(), qt.float().numpy()


def check(got, want, label):
    err = float(np.max(np.abs(got - want)))
    say(f"  {label}: max abs error {err:.2e}")
    assert np.all(np.isfinite(got)), label
    assert np.allclose(got, want, atol=0.006, rtol=0.025), (label, err)
    assert err < 3e-3, (label, err)


@pytest.mark.parametrize("heads,rpr", [(8, 1), (16, 2), (24, 1), (40, 4), (72, 2), (128, 1)])
def test_sparse_attention_paged_matches_oracle(torch_gpu, heads, rpr):
    torch = torch_gpu
    rng = np.random.default_rng(heads)
    say(f"case paged heads={heads} rows_per_request={rpr}")
    blocks, max_blocks, rows = 48, 24, 8
    batch = rows // rpr
    h_kv = np.concatenate([sfa.kv_payload(int(b % 5), np.arange(128) + b * 128) for b in range(blocks)])
    h_kv = h_kv.reshape(blocks, 128, ROW)
    table = np.stack([rng.permutation(blocks)[:max_blocks] for _ in range(batch)]).astype(np.int32)
    idx = rng.integers(0, max_blocks * 128, (rows, TOPK)).astype(np.int32)
    idx[rng.random((rows, TOPK)) < 0.2] = -1
    idx[1, 100:300] = idx[1, 0]  # a repeated position counts every time
    idx[rows - 1] = -1           # no valid index: zeros
    q, qh = bf16_query(torch, rng, rows, heads)
    out = sparse_attention(q, torch.from_numpy(h_kv).cuda(), torch.from_numpy(table).cuda(),
                           torch.from_numpy(idx).cuda(), SCALE, rows_per_request=rpr).cpu().numpy()
    want = np.zeros((rows, heads, 512), np.float32)
    for r in range(rows - 1):
        t = idx[r][idx[r] >= 0]
        want[r] = sfa.sparse_attention(qh[r], h_kv[table[r // rpr][t // 128], t % 128], SCALE)
    check(out, want, f"paged h{heads}")
    assert not out[rows - 1].any()


@pytest.mark.parametrize("heads,rows", [(16, 256), (128, 128)])
def test_sparse_attention_unsplit_rows_match_oracle(torch_gpu, heads, rows):
    """Enough rows that the launch fills the GPU without index splits: each workgroup
    normalises and writes its heads' output itself (no partials, no merge launch), for
    the 16-head kernel and for the kernel of four waves per 32 heads."""
    torch = torch_gpu
    rng = np.random.default_rng(heads + rows)
    say(f"case unsplit heads={heads} rows={rows}")
    blocks, max_blocks = 40, 20
    h_kv = np.concatenate([sfa.kv_payload(int(b % 3), np.arange(128) + b * 128) for b in range(blocks)])
    h_kv = h_kv.reshape(blocks, 128, ROW)
    table = np.stack([rng.permutation(blocks)[:max_blocks] for _ in range(rows)]).astype(np.int32)
    idx = rng.integers(0, max_blocks * 128, (rows, TOPK)).astype(np.int32)
    idx[rng.random((rows, TOPK)) < 0.75] = -1
    q, qh = bf16_query(torch, rng, rows, heads)
    out = sparse_attention(q, torch.from_numpy(h_kv).cuda(), torch.from_numpy(table).cuda(),
                           torch.from_numpy(idx).cuda(), SCALE).cpu().numpy()
    for r in range(rows):
        t = idx[r][idx[r] >= 0]
        want = sfa.sparse_attention(qh[r], h_kv[table[r][t // 128], t % 128], SCALE)
        if r % 32 == 0:
            say(f"  row {r}: max abs error {float(np.max(np.abs(out[r] - want))):.2e}")
        assert np.all(np.isfinite(out[r])), r
        assert np.allclose(out[r], want, atol=0.006, rtol=0.025), r
        assert float(np.max(np.abs(out[r] - want))) < 3e-3, r


def test_sparse_attention_reports_bad_positions(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(2)
    h_kv = sfa.kv_payload(0, np.arange(4 * 128)).reshape(4, 128, ROW)
    table = np.array([[0, 1, 2, 3], [3, 2, 1, 9]], np.int32)  # block 9 does not exist
    idx = rng.integers(0, 512, (2, TOPK)).astype(np.int32)
    idx[0, 5] = 512    # beyond the block table
    idx[1, :] = 400    # block 3 of request 1 -> 9: absent throughout
    q, qh = bf16_query(torch, rng, 2, 8)
    op = kvip_amd.SparseAttention(torch, rows=2, heads=8, device="cuda")
    op.bind(q, torch.from_numpy(h_kv).cuda(), torch.from_numpy(table).cuda(), torch.from_numpy(idx).cuda(), SCALE)
    out = op().cpu().numpy()
    torch.cuda.synchronize()
    status = int(op.status.item())
    assert status & abi_bits("BAD_TOKEN") and status & abi_bits("BAD_BLOCK"), status
    keep = np.delete(idx[0], 5)
    check(out[:1], sfa.sparse_attention(qh[0], h_kv[table[0][keep // 128], keep % 128], SCALE)[None], "bad-row")
    assert not out[1].any()


def abi_bits(name):
    from kvip_amd.runtime import abi
    return getattr(abi, f"STATUS_{name}")


def test_sparse_attention_on_gathered_rows(torch_gpu):
    torch = torch_gpu
    say("case gathered rows of the contiguous forward")
    wl = synthetic.decode_workload(torch, batch=4, ctx=[9000, 2100, 5000, 3000], device="cuda", seed=3)
    blocks = int(wl.kv_cache.shape[0])
    h_kv = np.concatenate([sfa.kv_payload(int(b % 7), np.arange(128) + b * 128) for b in range(blocks)])
    wl.kv_cache.copy_(torch.from_numpy(h_kv.reshape(blocks, 128, ROW)))
    rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
    fwd()
    torch.cuda.synchronize()
    kv, table, indices = gathered_table(torch, upd)
    rng = np.random.default_rng(9)
    q, qh = bf16_query(torch, rng, 4, 16)
    out = sparse_attention(q, kv, table, indices, SCALE).cpu().numpy()
    top = rot.topk.cpu().numpy()
    bt = wl.block_table.cpu().numpy()
    h_kv = h_kv.reshape(blocks, 128, ROW)
    want = np.stack([sfa.sparse_attention(qh[r], h_kv[bt[r][top[r] // 128], top[r] % 128], SCALE) for r in range(4)])
    check(out, want, "gathered")


def test_sparse_attention_on_resident_hot_cache(torch_gpu):
    """check_sfa (correctness.py:261-339): LI + TopK + resident round on the device, then
    attention over the hot cache at the slot outputs against the logical tokens' payload."""
    torch = torch_gpu
    say("case resident hot cache")
    batch, owners, history, resident, q_rows = 2, 2, 8192, 4096, 4
    rng = np.random.default_rng(21)
    keys = rng.integers(0, 256, (owners, history, 128), dtype=np.uint8) & 0x77
    pool = np.concatenate([sfa.kv_payload(o, np.arange(history)) for o in range(owners)])
    t, dev = torch, "cuda"
    pool_t = t.empty(pool.size, dtype=t.uint8, pin_memory=True)
    pool_t.copy_(t.from_numpy(pool.reshape(-1)))
    hot = t.from_numpy(np.stack([pool[o * history:o * history + resident] for o in range(owners)])).to(dev)
    rot = kvip_amd.LIFetchBinding(t, batch=batch, max_context=history, device=dev, heads=32, rows_per_request=q_rows,
                                  qk_dtype="fp8", query_ends=True)
    rot.seq_lens.fill_(history)
    rot.query_ends.copy_(t.arange(history - 3, history + 1, dtype=t.int32).repeat(batch))
    # The four MTP rows of a request share their LI query, so their selections overlap and
    # the misses fit the LRU candidates.
    q_li = np.repeat(rng.standard_normal((batch, 32, 128)).astype(np.float32), q_rows, axis=0)
    rot.query.copy_(t.from_numpy(q_li).to(t.float8_e4m3fn))
    rot.weights.copy_(t.from_numpy(np.repeat(rng.standard_normal((batch, 32)).astype(np.float32), q_rows, axis=0)))
    upd = kvip_amd.ResidentIndexUpdate(
        t, keys=t.from_numpy(keys).to(dev).view(t.float8_e4m3fn),
        scales=t.from_numpy(rng.uniform(0.5, 2.0, (owners, history)).astype(np.float32)).to(dev),
        addresses=t.from_numpy((np.arange(owners * history) * ROW).reshape(owners, history)).to(dev),
        logical_ids=t.arange(history, dtype=t.int64, device=dev).repeat(owners, 1).contiguous(),
        row_owners=t.arange(batch, dtype=t.int32, device=dev), rotating=rot,
        hot_valid=t.ones((owners, resident), dtype=t.int32, device=dev), hot_cache=hot, host_pool=pool_t,
        resident=resident)
    upd.set_candidates(t.from_numpy(np.stack([rng.permutation(resident)[:TOPK] for _ in range(batch)])
                                    .astype(np.int32)).to(dev))
    kvip_amd.LIFetch(rot, upd)()
    t.cuda.synchronize()
    assert not upd.status.any(), upd.status.cpu().tolist()
    kv, table = hot_cache_table(t, upd)
    q, qh = bf16_query(t, rng, batch * q_rows, 8)
    out = sparse_attention(q, kv, table, upd.slot_output.view(batch * q_rows, TOPK), SCALE,
                           rows_per_request=q_rows).cpu().numpy()
    logical = upd.logical_output.view(batch * q_rows, TOPK).cpu().numpy()
    assert (logical >= 0).all()
    want = np.stack([sfa.sparse_attention(qh[r], sfa.kv_payload(r // q_rows, logical[r]), SCALE)
                     for r in range(batch * q_rows)])
    check(out, want, "resident hot cache")


@pytest.mark.parametrize("heads", [16, 128])
def test_sparse_attention_graph_replay(torch_gpu, heads):
    """The split launch and its merge launch captured in a hipGraph (the 16-head kernel and
    the kernel of four waves per 32 heads): every replay, with eager work between replays,
    equals the eager call bit for bit, and so does an eager call after the replays."""
    torch = torch_gpu
    rng = np.random.default_rng(33)
    rows, blocks = 16, 40
    h_kv = np.concatenate([sfa.kv_payload(int(b % 3), np.arange(128) + b * 128) for b in range(blocks)])
    kv = torch.from_numpy(h_kv.reshape(blocks, 128, ROW)).cuda()
    table = torch.from_numpy(np.stack([rng.permutation(blocks)[:16] for _ in range(rows)]).astype(np.int32)).cuda()
    idx = torch.from_numpy(rng.integers(0, 16 * 128, (rows, TOPK)).astype(np.int32)).cuda()
    q, _ = bf16_query(torch, rng, rows, heads)
    op = kvip_amd.SparseAttention(torch, rows=rows, heads=heads, device="cuda").bind(q, kv, table, idx, SCALE)
    eager = op().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            op()
    torch.cuda.current_stream().wait_stream(side)
    for replay in range(3):
        op.output.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(op.output, eager), replay
        _ = (q.float() * 2).sum().item()  # eager work between replays
    op.output.zero_()
    assert torch.equal(op(), eager)
