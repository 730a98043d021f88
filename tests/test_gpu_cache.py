"""GPU parity of the cache operators (update_abc, SlotLRU) against oracle/cache.py,
bit-exact, through the C ABI."""
import numpy as np
import pytest

import kvip_amd
from kvip_amd.runtime import abi
from oracle import cache as ref

pytestmark = pytest.mark.gpu


def run_abc(torch, t2s, s2t, desc, requests, history, tail):
    dt2s, ds2t = torch.from_numpy(t2s).cuda(), torch.from_numpy(s2t).cuda()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    kvip_amd.update_abc(dt2s, ds2t, torch.from_numpy(desc).cuda(), requests, history, tail, status=status)
    torch.cuda.synchronize()
    ref.update_abc(t2s, s2t, desc, requests, history, tail)
    return dt2s.cpu().numpy(), ds2t.cpu().numpy(), int(status.item())


def test_update_abc_known_answer_and_shifted_rings(torch_gpu):
    torch = torch_gpu
    t2s = np.full((2, 3, 2048), -1, np.int32)
    s2t = t2s.copy()
    g2, g3, st = run_abc(torch, t2s, s2t, np.array([[[1, 2, 383, 390]]], np.int32), 1, 1024, 384)
    assert np.array_equal(g2, t2s) and np.array_equal(g3, s2t) and st == 0
    desc = np.array([[[2, 4, 350, 734], [2, 1, 768, 768]], [[0, 3, 383, 390], [0, 2, 128, 140]]], np.int32)
    t2s = np.full((3, 5, 2048), 99, np.int32)
    s2t = t2s.copy()
    dt2s, ds2t = torch.from_numpy(t2s).cuda(), torch.from_numpy(s2t).cuda()
    for shift in (0, 128):
        desc[:, :, 2:] += shift
        kvip_amd.update_abc(dt2s, ds2t, torch.from_numpy(desc).cuda(), 2, 1024, 384)
        ref.update_abc(t2s, s2t, desc, 2, 1024, 384)
        torch.cuda.synchronize()
        assert np.array_equal(dt2s.cpu().numpy(), t2s) and np.array_equal(ds2t.cpu().numpy(), s2t), shift


def test_update_abc_random_duplicates_long_and_empty_ranges(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(12)
    for trial in range(4):
        layers, pool, tokens, history, tail = 3, 4, 3000, 2000, 384
        groups, rows = int(rng.integers(1, 5)), int(rng.integers(1, 7))
        desc = np.zeros((groups, rows, 4), np.int32)
        desc[..., 0] = rng.integers(0, layers, (groups, rows))
        desc[..., 1] = rng.integers(0, 2, (groups, rows))  # few owners -> duplicate targets
        begin = rng.integers(0, 2500, (groups, rows))
        length = rng.choice([0, 5, 383, 384, 385, 1000], (groups, rows))
        desc[..., 2] = begin
        desc[..., 3] = np.minimum(begin + length, tokens)
        t2s = rng.integers(-3, 5000, (layers, pool, tokens)).astype(np.int32)
        s2t = rng.integers(-3, 5000, (layers, pool, tokens)).astype(np.int32)
        requests = int(rng.integers(1, rows + 1))
        g2, g3, st = run_abc(torch, t2s, s2t, desc, requests, history, tail)
        assert np.array_equal(g2, t2s), trial
        assert np.array_equal(g3, s2t), trial
        assert st == 0


def test_update_abc_rejects_and_reports(torch_gpu):
    torch = torch_gpu
    t2s = torch.zeros((1, 2, 512), dtype=torch.int32, device="cuda")
    s2t = torch.zeros((1, 2, 512), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        kvip_amd.update_abc(t2s.cpu(), s2t.cpu(), torch.zeros((1, 1, 4), dtype=torch.int32), 1, 100, 50)
    with pytest.raises(ValueError):
        kvip_amd.update_abc(t2s, s2t, torch.zeros((1, 1, 4), dtype=torch.int32, device="cuda"), 1, 500, 50)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    bad = torch.tensor([[[0, 7, 0, 10]]], dtype=torch.int32, device="cuda")  # owner out of range
    kvip_amd.update_abc(t2s, s2t, bad, 1, 100, 50, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & abi.STATUS_BAD_TOKEN
    assert not t2s.any() and not s2t.any()


def check_lru(torch, gpu, cpu):
    assert gpu.active == cpu.active
    assert gpu.slots.cpu().numpy()[0].tolist() == cpu.slots.tolist()
    words = cpu.bitmap.shape[0]
    assert np.array_equal(gpu.bitmap.cpu().numpy()[0][:words].view(np.uint32), cpu.bitmap)
    assert gpu.order[: gpu.active].cpu().numpy().tolist() == cpu.order()


def test_slot_lru_matches_oracle(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(9)
    gpu, cpu = kvip_amd.SlotLRU("cuda"), ref.SlotLRU()
    gpu.resize(16384, 16384)
    cpu.resize(16384, 16384)
    check_lru(torch, gpu, cpu)
    first = gpu.slots.clone()
    for step in range(40):
        if step in (10, 25):
            committed = int(rng.integers(1, 16384))
            gpu.resize(16384, committed)
            cpu.resize(16384, committed)
        elif step == 30:
            gpu.resize(40000, 30000)
            cpu.resize(40000, 30000)
        else:
            dest = rng.integers(-3, cpu.active + 20, int(rng.integers(0, 9000))).astype(np.int32)
            # Device int32 tensors, and the reference's host numpy call (int32 / int64).
            host = dest if step % 3 == 1 else dest.astype(np.int64)
            gpu.commit(host if step % 3 else torch.from_numpy(dest).cuda())
            cpu.commit(dest)
        torch.cuda.synchronize()
        check_lru(torch, gpu, cpu)
    assert not torch.equal(first, gpu.slots)
    gpu.resize(40000, 100)
    cpu.resize(40000, 100)
    torch.cuda.synchronize()
    check_lru(torch, gpu, cpu)
    assert (gpu.slots[0, 100:] == -1).all()


def test_slot_lru_chains_match_per_chain_oracles(torch_gpu):
    """SlotLRUChains (kvip_hip_lru_reset_chains / _commit_chains, one launch per batch)
    against one oracle SlotLRU per chain: destinations are rows of a wider buffer (row
    stride above the count) with -1 padding and out-of-range slots; the chains' slots
    alias a caller's candidate buffer; committing inside a captured hipGraph equals the
    eager commits."""
    torch = torch_gpu
    rng = np.random.default_rng(31)
    chains, capacity = 5, 6000
    cand = torch.full((chains, 2048), -7, dtype=torch.int32, device="cuda")
    gpu = kvip_amd.SlotLRUChains(torch, chains, capacity, "cuda", slots=cand)
    cpus = [ref.SlotLRU() for _ in range(chains)]
    for c in cpus:
        c.resize(capacity, capacity)

    def check():
        torch.cuda.synchronize()
        order = gpu.order.cpu().numpy()
        slots = cand.cpu().numpy()
        bitmap = gpu.bitmap.cpu().numpy()
        for k, c in enumerate(cpus):
            assert slots[k].tolist() == c.slots.tolist(), k
            assert order[k][:c.active].tolist() == c.order(), k
            assert (order[k][c.active:] == -1).all(), k
            assert np.array_equal(bitmap[k][:c.bitmap.shape[0]].view(np.uint32), c.bitmap), k

    check()
    buf = torch.full((chains, 3000), -1, dtype=torch.int32, device="cuda")
    for step in range(6):
        host = np.full((chains, 2500), -1, np.int32)
        for k in range(chains):
            n = int(rng.integers(0, 2500))
            host[k, :n] = rng.integers(-2, capacity + 10, n)
        buf[:, :2500].copy_(torch.from_numpy(host))
        gpu.commit(buf[:, :2500])
        for k, c in enumerate(cpus):
            c.commit(host[k])
        check()
    # Captured: the commit of a fixed buffer, replayed after the buffer is refilled.
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            gpu.commit(buf[:, :2500])
    torch.cuda.current_stream().wait_stream(side)
    for step in range(3):
        host = rng.integers(0, capacity, (chains, 2500)).astype(np.int32)
        buf[:, :2500].copy_(torch.from_numpy(host))
        graph.replay()
        for k, c in enumerate(cpus):
            c.commit(host[k])
        check()
    gpu.reset(100)
    for c in cpus:
        c.resize(capacity, 100)
    check()
    assert (cand[:, 100:] == -1).all()


def test_publish_pages_matches_oracle(torch_gpu):
    """PageUpdates.submit (kvip_hip_publish_pages) against oracle.cache.publish_pages over
    three submissions alternating the staging ring: addresses, validity, cleared map ranges
    and the fused per-group token-address tables bit-exact; a row with an out-of-range
    index is skipped and reported."""
    import kvip_amd
    from oracle.cache import publish_pages

    torch = torch_gpu
    rng = np.random.default_rng(17)
    owners, groups, pages, block, history = 5, 2, 24, 128, 3000  # history ends inside page 23
    widths = (1, 2)
    addresses = torch.zeros((owners, groups, pages), dtype=torch.int64, device="cuda")
    valid = torch.zeros((owners, groups, pages), dtype=torch.uint8, device="cuda")
    mapping = torch.arange(owners * 4096, dtype=torch.int32, device="cuda")
    fused = tuple(torch.zeros((owners, history), dtype=torch.int64, device="cuda") for _ in range(groups))
    pu = kvip_amd.PageUpdates(torch, addresses, valid, mapping, fused=fused, widths=widths)
    h_addr, h_valid, h_map = (t.cpu().numpy() for t in (addresses, valid, mapping))
    h_fused = tuple(t.cpu().numpy() for t in fused)
    for step in range(3):
        index = rng.choice(owners * groups * pages, 40, replace=False)
        rows = [(int(i), int(rng.integers(0, 1 << 40)) * 16, int(rng.integers(0, owners * 4096 - block))
                 if rng.random() < 0.5 else -1) for i in index]
        pu.submit(rows, step % 2)
        publish_pages(h_addr, h_valid, h_map, rows, block, h_fused, widths, 656)
    torch.cuda.synchronize()
    assert int(pu.status.item()) == 0
    assert np.array_equal(addresses.cpu().numpy(), h_addr)
    assert np.array_equal(valid.cpu().numpy(), h_valid)
    assert np.array_equal(mapping.cpu().numpy(), h_map)
    for got, want in zip(fused, h_fused):
        assert np.array_equal(got.cpu().numpy(), want)
    pu.submit([(owners * groups * pages, 5, -1)], 1)
    torch.cuda.synchronize()
    assert int(pu.status.item()) == 4  # KVIP_STATUS_BAD_TOKEN
    assert np.array_equal(addresses.cpu().numpy(), h_addr)
