"""GPU parity of kvip_amd.lidu (kvip_hip_lidu through the C ABI) against oracle/lidu.py:
every output, the three state tensors and the untouched entries, bit-exact."""
import numpy as np
import pytest

import kvip_amd
from oracle import lidu as ref
from tests import lidu_cases as lc

pytestmark = pytest.mark.gpu


def upload(torch, case):
    return {k: torch.from_numpy(np.ascontiguousarray(case[k])).cuda() for k in lc.INPUTS}


def device_outputs(torch, case):
    outs = lc.empty_outputs(case["topk"].shape[0], len(case["actual_seq_lengths_query"]))
    return {k: torch.from_numpy(v).cuda() for k, v in outs.items()}


def call(torch, dev, outs, case):
    batch = len(case["actual_seq_lengths_query"])
    profiling = torch.zeros((batch, 8, 32), dtype=torch.int64, device="cuda")
    kvip_amd.lidu(*[dev[k] for k in lc.INPUTS], *[outs[k] for k in lc.OUTPUTS], profiling, case["layer_id"],
                  case["num_layers"], case["max_num_reqs"], case["qcap"])
    return profiling


def compare(dev, outs, state, expect, tag):
    for k in lc.STATE:
        assert np.array_equal(dev[k].cpu().numpy(), state[k]), (tag, k)
    for k in lc.OUTPUTS:
        got = outs[k].cpu().numpy()
        if not np.array_equal(got, expect[k]):
            bad = np.argwhere(got.reshape(-1) != expect[k].reshape(-1))[:5].ravel()
            raise AssertionError(f"{tag} {k}: first mismatches at {bad.tolist()}: "
                                 f"{got.reshape(-1)[bad].tolist()} != {expect[k].reshape(-1)[bad].tolist()}")


def check_case(torch, case, tag):
    print(f"lidu case {tag}", flush=True)
    dev = upload(torch, case)
    outs = device_outputs(torch, case)
    call(torch, dev, outs, case)
    torch.cuda.synchronize()
    state, expect = lc.run_oracle(case)
    compare(dev, outs, state, expect, tag)
    return state, expect


@pytest.mark.parametrize("seed,queries,kw", [
    (1, (1, 2, 4), {}),
    (2, (4, 4), dict(hot_tokens=8192, hit_share=0.3, budget=8192)),
    (3, (3, 1, 2, 4), dict(cand=(1 << 20) + 1000, hot_tokens=4096)),
    (4, (2, 2), dict(trailing=3)),
    (5, (4,), dict(hot_tokens=2048, hit_share=1.0)),
    (6, (4, 2), dict(hot_tokens=8192, hit_share=0.0, budget=12288, cand=40000)),
    (10, (1,) * 16, dict(budget=(1 << 17) + 2560, cand=300000, hot_tokens=2500)),
    (12, (1, 2, 3, 4, 4, 3, 2, 1, 2, 4, 3), {}),  # 11 requests: a partial second group of 8
])
def test_lidu_matches_oracle(torch_gpu, seed, queries, kw):
    check_case(torch_gpu, lc.random_case(seed, queries=queries, **kw), f"seed{seed}")


def test_lidu_known_answers(torch_gpu):
    from tests.test_oracle_lidu import kat_fixture, set_victims

    torch = torch_gpu
    check_case(torch, kat_fixture(4096, 4096, padding_second_row=False), "kat-literal")
    case = kat_fixture(8192, 4096, padding_second_row=True)
    set_victims(case, 4096)
    state, expect = check_case(torch, case, "kat-adapted")
    assert expect["miss_counts"].tolist() == [0, 0, 0]
    history = 1 << 20
    t2s = np.full((2, history + 2560), -1, np.int32)
    t2s[:, :4096] = np.arange(4096, dtype=np.int32)
    case.update(token_to_slot=t2s, qcap=(history + 2560) // 128)
    case["candidate_lens"][0] = case["logical_seq_lengths"][0] = history
    tile = history // 4
    case["topk"][:] = np.concatenate([np.arange(e - 512, e, dtype=np.int32) for e in range(tile, history + 1, tile)])
    state, expect = check_case(torch, case, "kat-tiles")
    assert expect["miss_counts"].tolist() == [2048, 0, 2048]


def test_lidu_padding_errors_and_graph_dummy(torch_gpu):
    torch = torch_gpu
    case = lc.add_padding_row(lc.add_padding_row(lc.random_case(7, queries=(2, 1)), queries=2), queries=0)
    case["topk"][0, 0, :5] = [-1, -1, 5, case["candidate_lens"][0] + 3, -1]
    check_case(torch, case, "padding+bad-token")
    case["profile_enabled"][0] = ref.PROFILE_MODE_GRAPH_DUMMY
    check_case(torch, case, "graph-dummy")
    base = lc.random_case(8, queries=(2, 2, 2), hot_tokens=8192, hit_share=0.2, budget=6144)
    edits = {
        "metadata": lambda c: c["cache_tokens"].__setitem__(1, 2047),
        "destination": lambda c: c["miss_slots"].__setitem__((1, 3), c["cache_tokens"][1]),
        "resident_block": lambda c: c["resident_block_table"].__setitem__((1, slice(None)), -1),
        "insufficient": lambda c: (c["cache_tokens"].__setitem__(1, 2200),
                                   c["miss_slots"].__setitem__(1, np.arange(2048)),
                                   c["miss_slot_bitmap"].__setitem__(1, lc.bitmap_of(range(2048)))),
        "alias": lambda c: c["req_pool_entries"].__setitem__(2, c["req_pool_entries"][0]),
        "too_many": lambda c: c["actual_seq_lengths_query"].__setitem__(slice(None), [5, 6, 6]),
        "empty_row": lambda c: c["actual_seq_lengths_query"].__setitem__(1, c["actual_seq_lengths_query"][0]),
    }
    for name, edit in edits.items():
        case = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in base.items()}
        edit(case)
        check_case(torch, case, name)


def test_lidu_extended_selection_and_profiling(torch_gpu):
    torch = torch_gpu
    case = lc.random_case(11, queries=(4, 4, 3), hot_tokens=8192, hit_share=0.25, budget=8192, cand=65536)
    dev = upload(torch, case)
    outs = device_outputs(torch, case)
    dev["profile_enabled"].fill_(1)
    case["profile_enabled"][0] = 1
    profiling = call(torch, dev, outs, case)
    torch.cuda.synchronize()
    state, expect = lc.run_oracle(case)
    assert (expect["miss_counts"][:-1] > 2048).any()
    compare(dev, outs, state, expect, "extended")
    stamps = profiling[:, 0, :9].cpu().numpy()
    assert (stamps > 0).all() and (np.diff(stamps, axis=1) >= 0).all()
    assert not profiling[:, 1:].any()


def test_lidu_rounds_evolve_state_eagerly_and_in_a_graph(torch_gpu):
    """Three eager rounds, then the same call captured once and replayed with new TopK
    rows; every round is checked against the oracle run on the previous round's state."""
    torch = torch_gpu
    case = lc.random_case(12, queries=(2, 4, 1), hot_tokens=6000, hit_share=0.5, budget=8192, cand=50000)
    rng = np.random.default_rng(5)
    dev = upload(torch, case)
    outs = device_outputs(torch, case)

    def next_topk():
        for q in range(case["topk"].shape[0]):
            r = int(np.searchsorted(case["actual_seq_lengths_query"], q, side="right"))
            cand = int(case["candidate_lens"][r])
            case["topk"][q, 0] = rng.choice(cand, 2048, replace=False)

    def step(run, tag):
        expect_state, expect = lc.run_oracle(case)
        for k, v in lc.empty_outputs(*case["topk"].shape[:1], len(case["actual_seq_lengths_query"])).items():
            outs[k].copy_(torch.from_numpy(v))
        run()
        torch.cuda.synchronize()
        compare(dev, outs, expect_state, expect, tag)
        for k in lc.STATE:
            case[k] = expect_state[k]

    for i in range(3):
        next_topk()
        dev["topk"].copy_(torch.from_numpy(case["topk"]))
        step(lambda: call(torch, dev, outs, case), f"eager{i}")
    profiling = torch.zeros((3, 8, 32), dtype=torch.int64, device="cuda")
    args = [dev[k] for k in lc.INPUTS] + [outs[k] for k in lc.OUTPUTS] + [profiling, case["layer_id"],
                                                                          case["num_layers"], case["max_num_reqs"],
                                                                          case["qcap"]]
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # Capture records the launches only; state and outputs are untouched until replay.
        snapshot = {k: dev[k].clone() for k in lc.STATE}
        with torch.cuda.graph(graph, stream=stream):
            kvip_amd.lidu(*args)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for k in lc.STATE:
        assert torch.equal(dev[k], snapshot[k])
    for i in range(3):
        next_topk()
        dev["topk"].copy_(torch.from_numpy(case["topk"]))
        step(graph.replay, f"replay{i}")


def test_lidu_prepare_allocating_variant(torch_gpu):
    torch = torch_gpu
    case = lc.random_case(13, queries=(2, 3))
    dev = upload(torch, case)
    res = kvip_amd.lidu_prepare(*[dev[k] for k in lc.INPUTS], case["layer_id"], case["num_layers"],
                                case["max_num_reqs"], case["qcap"])
    torch.cuda.synchronize()
    state, expect = lc.run_oracle(case)
    total = int(expect["miss_counts"][-1])
    for k, got in zip(lc.OUTPUTS, res):
        got = got.cpu().numpy()
        want = expect[k]
        if k in ("indices", "offsets", "output_indices"):
            got, want = got[:total], want[:total]
        assert np.array_equal(got, want), k


def test_torch_op_out_variant_in_a_graph_matches_oracle(torch_gpu):
    """torch.ops.nanovllm_dsa.lidu_fused_batch_get_prepare_mtp_out (the registered operator the
    reference's harness looks up) with the workspace reserved at bind time: captured in a
    hipGraph before any eager call, then replayed on fresh TopK rows; every replay is checked
    against the oracle run on the previous round's state."""
    torch = torch_gpu
    case = lc.random_case(21, queries=(4, 1, 3), hot_tokens=5000, hit_share=0.6, budget=8192, cand=60000)
    rng = np.random.default_rng(9)
    dev = upload(torch, case)
    outs = device_outputs(torch, case)
    batch = len(case["actual_seq_lengths_query"])
    kvip_amd.lidu_reserve("cuda", max_batch=8)
    profiling = torch.zeros((batch, 8, 32), dtype=torch.int64, device="cuda")
    op = torch.ops.nanovllm_dsa.lidu_fused_batch_get_prepare_mtp_out
    args = [dev[k] for k in lc.INPUTS] + [outs[k] for k in lc.OUTPUTS] + [profiling, case["layer_id"],
                                                                          case["num_layers"], case["max_num_reqs"],
                                                                          case["qcap"]]
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            res = op(*args)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert all(r.data_ptr() == outs[k].data_ptr() for r, k in zip(res, lc.OUTPUTS))
    for i in range(3):
        for q in range(case["topk"].shape[0]):
            r = int(np.searchsorted(case["actual_seq_lengths_query"], q, side="right"))
            case["topk"][q, 0] = rng.choice(int(case["candidate_lens"][r]), 2048, replace=False)
        dev["topk"].copy_(torch.from_numpy(case["topk"]))
        expect_state, expect = lc.run_oracle(case)
        for k, v in lc.empty_outputs(case["topk"].shape[0], batch).items():
            outs[k].copy_(torch.from_numpy(v))
        graph.replay()
        torch.cuda.synchronize()
        compare(dev, outs, expect_state, expect, f"op replay{i}")
        for k in lc.STATE:
            case[k] = expect_state[k]
