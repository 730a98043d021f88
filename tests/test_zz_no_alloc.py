"""GPU check of the allocation-free decode round (kvip_hip_lifetch_forward_static) through
the C ABI: on the same inputs it returns what kvip_hip_lifetch_forward returns (TopK ids
and gathered KV rows bit-exact, no status bits), on two calls in a row, the second with a
smaller batch and shorter rows (it reuses the library's scratch that the first left);
arguments that would need more than the library's scratch, or that pass their own
scratch, are rejected before anything runs."""
import ctypes

import pytest
import torch as _torch_module  # noqa: F401  (loads torch's HIP runtime before the library)

import kvip_amd
from kvip_amd import synthetic
from kvip_amd.runtime import abi

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)


def static_args(fwd):
    """The forward's arguments with every scratch pointer cleared."""
    a = abi.LIFetchArgs.from_buffer_copy(fwd.args)
    a.indexer.score_keys = 0
    a.indexer.histogram = 0
    a.topk.score_keys = 0
    a.topk.histogram = 0
    a.topk.segments = 0
    return a


def test_static_forward_equals_forward_on_two_calls(torch_gpu):
    torch = torch_gpu
    lib = abi.load_library()
    cases = [("batch 64 ctx U[8192,32768]", dict(batch=64, ctx_low=8192, ctx_high=32768, max_context=32768, seed=5)),
             ("batch 6 ctx U[1000,12000]", dict(batch=6, ctx_low=1000, ctx_high=12000, seed=6))]
    for name, kw in cases:
        say(f"case static forward {name}")
        wl = synthetic.decode_workload(torch, device="cuda", **kw)
        rot, upd, fwd = synthetic.bind(torch, kvip_amd, wl)
        fwd()
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        want_topk, want_rows = rot.topk.clone(), upd.output.clone()
        rot.topk.fill_(-9)
        upd.output.fill_(0xAB)
        args = static_args(fwd)
        rc = lib.kvip_hip_lifetch_forward_static(ctypes.byref(args), abi.stream_handle(torch, rot.device))
        assert rc == abi.KVIP_OK, rc
        torch.cuda.synchronize()
        assert int(rot.status.item()) == 0
        assert torch.equal(rot.topk, want_topk), name
        assert torch.equal(upd.output, want_rows), name
    # Rejected before anything runs: scratch beyond the library's array, or caller scratch.
    big = static_args(fwd)
    big.indexer.key_stride = big.topk.key_stride = (abi.LIFETCH_STATIC_SCRATCH_BYTES // (2 * 6)) // 8 * 8 + 8
    big.indexer.max_blocks = 1
    assert lib.kvip_hip_lifetch_forward_static(ctypes.byref(big), abi.stream_handle(torch, rot.device)) == \
        abi.KVIP_ERR_INVALID
    own = abi.LIFetchArgs.from_buffer_copy(fwd.args)
    assert lib.kvip_hip_lifetch_forward_static(ctypes.byref(own), abi.stream_handle(torch, rot.device)) == \
        abi.KVIP_ERR_INVALID
