"""The adapter oracle (oracle/adapters.py) against the known answers of the reference's
tests/adapters/test_inputs.py (values restated here), and the product's host-side
QueryInputs.prepare / validation on the CPU (its device work needs the GPU)."""
import numpy as np
import pytest

from oracle import adapters as ref


def test_mixed_query_counts_and_padding_kat():
    # test_inputs.py:30-41
    meta = ref.prepare_metadata(3, [1, 4])
    ends = ref.bind_positions(meta, np.array([57, 10000, 10001, 10002, 10003]))
    assert ends.reshape(3, 4).tolist() == [[58, 0, 0, 0], [10001, 10002, 10003, 10004], [0, 0, 0, 0]]
    query = np.repeat(np.arange(5, dtype=np.uint8)[:, None, None], 64, 1).repeat(128, 2)
    q, w, s = ref.pack(meta, query, np.arange(5.0)[:, None].repeat(64, 1), np.arange(5.0)[:, None].repeat(64, 1))
    assert q[:, 0, 0].tolist() == [0, 0, 0, 0, 1, 2, 3, 4, 0, 0, 0, 0]
    assert np.array_equal(w, s)
    assert meta[2, :5].tolist() == [0, 4, 5, 6, 7]
    assert meta[3, :8].tolist() == [1, 1, 1, 1, 1, 0, 0, 0]


def test_replay_and_rollback_kat():
    # test_inputs.py:43-54
    meta = ref.prepare_metadata(2, [2, 1])
    assert ref.bind_positions(meta, np.array([301, 302, 501])).reshape(2, 4).tolist() == [[302, 303, 0, 0],
                                                                                         [502, 0, 0, 0]]
    assert not ref.bind_positions(ref.prepare_metadata(2, [0, 0]), np.array([0])).any()


def test_owner_mapping_and_byte_gather_kat():
    # test_inputs.py:12-28, :89-97
    meta = ref.prepare_metadata(3, [1, 2], starts=[10, 20], owners=[7, 3])
    assert meta[4].view(np.int32)[:3].tolist() == [7, 3, 0]
    assert meta[0].tolist() == [10, 0, 0, 0, 20, 21, 0, 0, 0, 0, 0, 0]
    assert ref.prepare_metadata(3, [1], owners=[2])[4].view(np.int32)[:3].tolist() == [2, 0, 0]
    for heads in (32, 64):
        raw = (np.arange(3 * heads * 128) % 256).astype(np.uint8).reshape(3, heads, 128)
        q, _, _ = ref.pack(ref.prepare_metadata(2, [1, 2]), raw, np.ones((3, heads)), np.ones((3, heads)))
        assert np.array_equal(q, raw[[0, 0, 0, 0, 1, 2, 0, 0]])


def storage_cache():
    # test_inputs.py:148-154: 4 blocks of 2 tokens, row t filled with t, scale t.
    keys = np.repeat(np.arange(8, dtype=np.uint8)[:, None], 128, 1)
    return np.zeros((3, 32, 128), np.uint8), np.ones((3, 32), np.float32), keys, np.arange(8, dtype=np.float32)


def test_prefix_import_once_kat():
    # test_inputs.py:156-166
    keys, scales, src_k, src_s = storage_cache()
    imported = set()
    plan = (1, 2, 0, 2)  # owner, start, begin, stop
    ref.ingest_prefill(keys, scales, src_k, src_s, np.array([[2, 0]]), 2, np.array([0, 1]), [plan],
                       np.array([2, 3]), imported)
    assert keys[1, :4, 0].tolist() == [4, 5, 0, 1]
    assert scales[1, :4].tolist() == [4, 5, 0, 1]
    keys[1, 0] = 123
    ref.ingest_prefill(keys, scales, src_k, src_s, np.array([[2, 0]]), 2, np.array([0, 1]), [plan],
                       np.array([2, 3]), imported)
    assert keys[1, 0, 0] == 123


def test_decode_dynamic_owners_kat():
    # test_inputs.py:181-195
    keys, scales, src_k, src_s = storage_cache()
    keys[1:] = 99
    meta = ref.prepare_metadata(2, [1, 1])
    ends = ref.bind_positions(meta, np.array([4, 5]))
    ref.ingest_decode(keys, scales, src_k, src_s, np.array([6, 7]), meta, ends, np.array([1, 2]), 32)
    assert keys[1, 4, 0] == 6 and keys[2, 5, 0] == 7
    assert (keys[1:, :4] == 99).all()
    ends = ref.bind_positions(meta, np.array([3, 4]))
    ref.ingest_decode(keys, scales, src_k, src_s, np.array([6, 7]), meta, ends, np.array([2, 1]), 32)
    assert keys[2, 3, 0] == 6 and keys[1, 4, 0] == 7
    assert (keys[1:, :3] == 99).all()


def test_query_inputs_host_packing_matches_oracle_on_cpu():
    torch = pytest.importorskip("torch")
    from kvip_amd.adapters.vllm.inputs import QueryInputs

    rng = np.random.default_rng(4)
    inputs = QueryInputs(torch, 6, "cpu", pin_memory=False, history=512)
    pointers = (inputs.metadata.data_ptr(), inputs.query.data_ptr(), inputs.block_table.data_ptr())
    for trial in range(5):
        counts = [int(c) for c in rng.integers(0, 5, int(rng.integers(1, 7)))]
        starts = [int(s) for s in rng.integers(0, 1000, len(counts))] if trial % 2 else None
        owners = [int(o) for o in rng.integers(0, 50, len(counts))]
        inputs.prepare(counts, query_starts=starts, query_owners=owners)
        assert np.array_equal(inputs.metadata.numpy(), ref.prepare_metadata(6, counts, starts, owners)), trial
        want = np.array(owners + [0] * (6 - len(owners)))[:, None] * 4 + np.arange(4)
        assert np.array_equal(inputs.block_table.numpy(), want)
    assert pointers == (inputs.metadata.data_ptr(), inputs.query.data_ptr(), inputs.block_table.data_ptr())
    for counts in ([5], [1] * 7, [-1], [True]):
        with pytest.raises(ValueError):
            inputs.prepare(counts)
    with pytest.raises(ValueError):
        inputs.pack(torch.zeros(4, 32, 128), torch.zeros(4, 64), None)
    with pytest.raises(ValueError, match="GPU"):
        inputs.bind_positions(torch.zeros(3, dtype=torch.int64))


def test_committed_candidates():
    from kvip_amd.adapters.vllm.inputs import committed_candidates

    cands = np.array([9, 1, 7, 3, 0, 12], np.int32)
    assert committed_candidates(cands, 100, 16) is cands
    assert committed_candidates(cands, 5, 16).tolist() == [1, 3, 0, 2, 4, 9]


def test_token_order_publication_round_trips_pack():
    """publish_outputs undoes pack: a row computed from each packed query, published in
    token order, comes back to the token that query came from (decode-only batches, where
    the gather indices are the tokens themselves), and every other output row is -1."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        batch = int(rng.integers(1, 9))
        counts = [int(c) for c in rng.integers(0, 5, batch)]
        meta = ref.prepare_metadata(batch, counts)
        tokens = sum(counts)
        token_rows = rng.integers(0, 1 << 30, (max(tokens, 1), 7))
        packed = np.full((batch * 4, 7), -5, np.int64)
        valid = meta[1] != 0
        packed[valid] = token_rows[meta[0][valid]]
        out = ref.publish_outputs(meta, packed)
        assert np.array_equal(out[:tokens], token_rows[:tokens]), trial
        assert (out[tokens:] == -1).all(), trial


def test_token_order_publication_kat():
    # Counts [1, 4] of a batch of 3 (the known answer of test_inputs.py:30-41): tokens
    # 0..4 come from query rows 0, 4, 5, 6, 7; output rows 5..11 hold no token.
    meta = ref.prepare_metadata(3, [1, 4])
    rows = np.arange(12)[:, None] * 10 + np.arange(3)[None, :]
    out = ref.publish_outputs(meta, rows)
    assert out[:5, 0].tolist() == [0, 40, 50, 60, 70]
    assert (out[5:] == -1).all()


def test_binding_reads_query_inputs_on_cpu():
    """LIFetchBinding.bind_query_inputs swaps in the packed buffers of QueryInputs and
    refuses bindings whose shape or dtypes differ (host logic only)."""
    torch = pytest.importorskip("torch")
    import kvip_amd

    inputs = kvip_amd.QueryInputs(torch, 3, "cpu", pin_memory=False, history=512)
    rot = kvip_amd.LIFetchBinding(torch, batch=3, max_context=512, device="cpu", rows_per_request=4,
                                  weight_dtype=torch.bfloat16, query_ends=True).bind_query_inputs(inputs)
    for mine, theirs in ((rot.query, inputs.query), (rot.weights, inputs.weights), (rot.query_scale, inputs.scale),
                         (rot.query_ends, inputs.query_ends)):
        assert mine.data_ptr() == theirs.data_ptr()
    assert rot.seq_lens.tolist() == [512] * 3
    for kwargs in (dict(rows_per_request=1), dict(weight_dtype=torch.float32), dict(query_ends=False),
                   dict(heads=32), dict(batch=2)):
        args = dict(batch=3, max_context=512, device="cpu", rows_per_request=4, weight_dtype=torch.bfloat16,
                    query_ends=True)
        args.update(kwargs)
        with pytest.raises(ValueError):
            kvip_amd.LIFetchBinding(torch, **args).bind_query_inputs(inputs)
