"""GPU parity of the vLLM adapter's device work (kvip_hip_pack_queries,
kvip_hip_ingest_index through the C ABI): the reference's known answers
(tests/adapters/test_inputs.py) on the device and seeded random batches against
oracle/adapters.py, bit-exact."""
from types import SimpleNamespace as NS

import numpy as np
import pytest

from kvip_amd.adapters.vllm.index_import import VllmIndexCacheStorage
from kvip_amd.adapters.vllm.inputs import QueryInputs
from oracle import adapters as ref

pytestmark = pytest.mark.gpu


def test_query_inputs_known_answers(torch_gpu):
    torch = torch_gpu
    inputs = QueryInputs(torch, 3, "cuda")
    inputs.prepare([1, 4])
    ends = inputs.bind_positions(torch.tensor([57, 10000, 10001, 10002, 10003], device="cuda"))
    assert ends.tolist() == [[58, 0, 0, 0], [10001, 10002, 10003, 10004], [0, 0, 0, 0]]
    query = torch.arange(5).float()[:, None, None].expand(-1, 64, 128).to(torch.float8_e4m3fn).cuda()
    weights = torch.arange(5).bfloat16()[:, None].expand(-1, 64).contiguous().cuda()
    scale = torch.arange(5).float()[:, None].expand(-1, 64).contiguous().cuda()
    q, w, s = inputs.pack(query.contiguous(), weights, scale)
    assert q[:, 0, 0].float().tolist() == [0, 0, 0, 0, 1, 2, 3, 4, 0, 0, 0, 0]
    assert torch.equal(w.float(), s)
    assert inputs.unpack_indices[:5].tolist() == [0, 4, 5, 6, 7]
    # Rollback keeps every buffer address.
    pointers = (inputs.metadata.data_ptr(), inputs.query_ends.data_ptr(), inputs.query.data_ptr())
    inputs.prepare([2, 1])
    assert inputs.bind_positions(torch.tensor([301, 302, 501], device="cuda")).tolist()[:2] == [[302, 303, 0, 0],
                                                                                               [502, 0, 0, 0]]
    assert pointers == (inputs.metadata.data_ptr(), inputs.query_ends.data_ptr(), inputs.query.data_ptr())
    for heads in (32, 64):  # byte gather keeps every fp8 bit pattern, NaNs included
        inputs = QueryInputs(torch, 2, "cuda", index_heads=heads)
        inputs.prepare([1, 2])
        raw = torch.arange(3 * heads * 128).remainder(256).to(torch.uint8).reshape(3, heads, 128).cuda()
        packed, _, _ = inputs.pack(raw.view(torch.float8_e4m3fn), torch.ones(3, heads, dtype=torch.bfloat16).cuda(),
                                   torch.ones(3, heads).cuda())
        assert torch.equal(packed.view(torch.uint8), raw[[0, 0, 0, 0, 1, 2, 0, 0]])
        flat, _, s = inputs.pack(raw.view(torch.float8_e4m3fn).view(3 * heads, 128),
                                 torch.ones(3, heads, dtype=torch.bfloat16).cuda(),
                                 torch.arange(3 * heads).float().cuda())
        assert torch.equal(s.cpu(), torch.arange(3 * heads).float().view(3, heads)[[0, 0, 0, 0, 1, 2, 0, 0]])
    assert int(inputs.status.item()) == 0


def test_query_inputs_random_against_oracle(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(9)
    inputs = QueryInputs(torch, 16, "cuda")
    for trial in range(6):
        counts = [int(c) for c in rng.integers(0, 5, int(rng.integers(1, 17)))]
        tokens = max(1, sum(counts))
        starts = None
        if trial % 2:
            starts = [int(s) for s in rng.integers(0, tokens, len(counts))]
            starts = [min(s, tokens - c) if c else s for s, c in zip(starts, counts)]
        inputs.prepare(counts, query_starts=starts)
        meta = ref.prepare_metadata(16, counts, starts)
        positions = rng.integers(0, 1 << 20, tokens).astype(np.int64)
        query = rng.integers(0, 256, (tokens, 64, 128), dtype=np.uint8)
        weights = rng.standard_normal((tokens, 64)).astype(np.float32)
        scale = rng.standard_normal((tokens, 64)).astype(np.float32)
        ends = inputs.bind_positions(torch.from_numpy(positions).cuda())
        wt = torch.from_numpy(weights).bfloat16().cuda()
        q, w, s = inputs.pack(torch.from_numpy(query).cuda().view(torch.float8_e4m3fn), wt, torch.from_numpy(scale).cuda())
        want_q, want_w, want_s = ref.pack(meta, query, wt.cpu().view(torch.int16).numpy(), scale)
        assert np.array_equal(ends.cpu().numpy().reshape(-1), ref.bind_positions(meta, positions)), trial
        assert np.array_equal(q.view(torch.uint8).cpu().numpy(), want_q), trial
        assert np.array_equal(w.view(torch.int16).cpu().numpy(), want_w), trial
        assert np.array_equal(s.cpu().numpy(), want_s), trial
    assert int(inputs.status.item()) == 0


def device_cache(torch):
    keys = torch.arange(8, dtype=torch.uint8)[:, None].expand(-1, 128).clone().view(4, 2, 1, 128).cuda()
    return keys, torch.arange(8).float().view(4, 2, 1).cuda()


def test_index_storage_known_answers(torch_gpu):
    torch = torch_gpu
    storage = VllmIndexCacheStorage(torch, 3, 32, 8, "cuda")
    cache = device_cache(torch)
    plan = NS(owner=1, request="a", start=2, begin=0, stop=2)
    metadata = NS(block_size=2, block_table=torch.tensor([[2, 0]], device="cuda"),
                  slot_mapping=torch.tensor([0, 1], device="cuda"))
    storage.prepare([plan])
    storage.ingest_prefill(cache, metadata, [plan], torch.tensor([2, 3], device="cuda"))
    assert storage.keys[1, :4, 0].tolist() == [4, 5, 0, 1]
    assert storage.scales[1, :4].tolist() == [4, 5, 0, 1]
    storage.keys[1, 0].fill_(123)
    storage.prepare([plan])
    storage.ingest_prefill(cache, metadata, [plan], torch.tensor([2, 3], device="cuda"))
    assert int(storage.keys[1, 0, 0]) == 123
    # Decode: dynamic owners and corrected positions move only B*Q rows.
    storage = VllmIndexCacheStorage(torch, 3, 32, 8, "cuda")
    inputs = QueryInputs(torch, 2, "cuda")
    inputs.prepare([1, 1])
    inputs.bind_positions(torch.tensor([4, 5], device="cuda"))
    owners = torch.tensor([1, 2], dtype=torch.int32, device="cuda")
    metadata = NS(slot_mapping=torch.tensor([6, 7], device="cuda"))
    storage.keys[1:].fill_(99)
    storage.ingest_decode(cache, metadata, inputs, owners)
    assert int(storage.keys[1, 4, 0]) == 6 and int(storage.keys[2, 5, 0]) == 7
    assert bool(torch.all(storage.keys[1:, :4] == 99))
    owners.copy_(torch.tensor([2, 1], dtype=torch.int32))
    inputs.bind_positions(torch.tensor([3, 4], device="cuda"))
    storage.ingest_decode(cache, metadata, inputs, owners)
    assert int(storage.keys[2, 3, 0]) == 6 and int(storage.keys[1, 4, 0]) == 7
    assert bool(torch.all(storage.keys[1:, :3] == 99))
    assert int(storage.status.item()) == 0


def test_index_ingest_random_against_oracle(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(21)
    owners_n, history, blocks, block = 6, 4096, 300, 16
    src_k = rng.integers(0, 256, (blocks * block, 128), dtype=np.uint8)
    src_s = rng.standard_normal(blocks * block).astype(np.float32)
    cache = (torch.from_numpy(src_k).cuda().view(blocks, block, 1, 128), torch.from_numpy(src_s).cuda().view(blocks, block, 1))
    storage = VllmIndexCacheStorage(torch, owners_n, history, 64, "cuda")
    keys = np.zeros((owners_n, history, 128), np.uint8)
    scales = np.ones((owners_n, history), np.float32)
    imported = set()
    # Prefill: three requests with restored prefixes and current chunks.
    plans, tables, slot_list, pos_list, begin = [], [], [], [], 0
    for row, owner in enumerate((3, 1, 4)):
        start = int(rng.integers(0, 1000))
        n = int(rng.integers(1, 300))
        plans.append(NS(owner=owner, request=f"r{row}", start=start, begin=begin, stop=begin + n))
        tables.append(rng.choice(blocks, history // block, replace=False))
        slot_list.append(rng.choice(blocks * block, n, replace=False))
        pos_list.append(start + np.arange(n))
        begin += n
    table = np.stack(tables).astype(np.int32)
    slots = np.concatenate(slot_list).astype(np.int64)
    positions = np.concatenate(pos_list).astype(np.int64)
    storage.prepare(plans)
    metadata = NS(block_size=block, block_table=torch.from_numpy(table).cuda(), slot_mapping=torch.from_numpy(slots).cuda())
    storage.ingest_prefill(cache, metadata, plans, torch.from_numpy(positions).cuda())
    ref.ingest_prefill(keys, scales, src_k, src_s, table, block, slots,
                       [(p.owner, p.start, p.begin, p.stop) for p in plans], positions, imported)
    torch.cuda.synchronize()
    assert np.array_equal(storage.keys.cpu().numpy(), keys)
    assert np.array_equal(storage.scales.cpu().numpy(), scales)
    # Decode rounds with MTP counts, padding rows and changing owners.
    inputs = QueryInputs(torch, 4, "cuda")
    for trial in range(4):
        counts = [int(c) for c in rng.integers(1, 5, 3)]
        tokens = sum(counts)
        inputs.prepare(counts)
        meta = ref.prepare_metadata(4, counts)
        pos = rng.integers(8, history - 8, tokens).astype(np.int64)
        owners = rng.choice(np.arange(1, owners_n), 4, replace=False).astype(np.int32)
        slot_map = rng.choice(blocks * block, tokens, replace=False).astype(np.int64)
        inputs.bind_positions(torch.from_numpy(pos).cuda())
        storage.ingest_decode(cache, NS(slot_mapping=torch.from_numpy(slot_map).cuda()), inputs,
                              torch.from_numpy(owners).cuda())
        ref.ingest_decode(keys, scales, src_k, src_s, slot_map, meta, ref.bind_positions(meta, pos), owners, history)
        torch.cuda.synchronize()
        assert np.array_equal(storage.keys.cpu().numpy(), keys), trial
        assert np.array_equal(storage.scales.cpu().numpy(), scales), trial
    assert int(storage.status.item()) == 0
