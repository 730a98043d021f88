"""C ABI: the library loads on the CPU, exports every declared symbol, the ctypes
structs match the C layout, and invalid arguments are rejected before any launch."""
import ctypes
import re
import subprocess
import textwrap

import pytest

from kvip_amd.runtime import abi
from tests.conftest import ROOT

HEADER = ROOT / "include" / "kvip_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*uint(?:32|64)_t\s+(kvip_hip_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = abi.load_library()
    names = declared_functions()
    assert names, "no entry points parsed from the header"
    for name in names:
        assert hasattr(lib, name), name
        assert name in abi.PROTOTYPES, f"{name} has no ctypes prototype"
    assert set(abi.PROTOTYPES) == set(names)
    assert lib.kvip_hip_abi_version() == abi.ABI_VERSION


STRUCTS = {
    "KvipIndexerArgs": abi.IndexerArgs,
    "KvipPrefillArgs": abi.PrefillArgs,
    "KvipTopkArgs": abi.TopkArgs,
    "KvipFetchArgs": abi.FetchArgs,
    "KvipLIFetchArgs": abi.LIFetchArgs,
    "KvipAbcArgs": abi.AbcArgs,
    "KvipLruArgs": abi.LruArgs,
    "KvipLiduArgs": abi.LiduArgs,
    "KvipQueryPackArgs": abi.QueryPackArgs,
    "KvipIngestArgs": abi.IngestArgs,
    "KvipResidentArgs": abi.ResidentArgs,
    "KvipPrefixClassifyArgs": abi.PrefixClassifyArgs,
    "KvipPrefetchArgs": abi.PrefetchArgs,
    "KvipPageArgs": abi.PageArgs,
    "KvipSparseAttnArgs": abi.SparseAttnArgs,
}


def test_every_declared_struct_has_a_checked_layout():
    declared = set(re.findall(r"typedef struct (\w+)", (ROOT / "include" / "kvip_hip.h").read_text()))
    assert declared == set(STRUCTS)


def test_ctypes_layout_matches_c(tmp_path):
    lines = []
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    src = tmp_path / "layout.c"
    src.write_text(textwrap.dedent(
        '#include <stddef.h>\n#include <stdio.h>\n#include "kvip_hip.h"\nint main(void){\n'
        + "\n".join(lines) + "\nreturn 0;}\n"))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    c_layout = {(a, b): int(c) for a, b, c in (line.split() for line in out if line)}
    for cname, cls in STRUCTS.items():
        assert c_layout[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert c_layout[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_invalid_arguments_rejected_before_launch():
    lib = abi.load_library()
    assert lib.kvip_hip_indexer_decode(None, None) == abi.KVIP_ERR_INVALID
    assert lib.kvip_hip_topk(None, None) == abi.KVIP_ERR_INVALID
    assert lib.kvip_hip_fetch_gather(None, None) == abi.KVIP_ERR_INVALID
    assert lib.kvip_hip_lifetch_forward(None, None) == abi.KVIP_ERR_INVALID
    # Well-formed pointers but an unsupported head count / unaligned key stride.
    args = abi.IndexerArgs(query=16, weights=16, keys=16, block_table=16, seq_lens=16, score_keys=16,
                           histogram=16, key_block_stride=16384, batch=1, rows_per_request=1, heads=48,
                           max_blocks=1, num_blocks=1, key_stride=128, qk_dtype=abi.DTYPE_FP8_E4M3,
                           weight_dtype=abi.DTYPE_FP32)
    assert lib.kvip_hip_indexer_decode(ctypes.byref(args), None) == abi.KVIP_ERR_INVALID
    args.heads = 64
    args.key_stride = 100
    assert lib.kvip_hip_indexer_decode(ctypes.byref(args), None) == abi.KVIP_ERR_INVALID
    topk = abi.TopkArgs(score_keys=16, seq_lens=16, topk=16, batch=1, rows_per_request=3, key_stride=128)
    assert lib.kvip_hip_topk(ctypes.byref(topk), None) == abi.KVIP_ERR_INVALID
    fetch = abi.FetchArgs(topk=16, kv_cache=16, block_table=16, output=16, kv_block_stride=128 * 656,
                          row_stride=656, row_bytes=650, batch=1, rows_per_request=1, max_blocks=1, num_blocks=1)
    assert lib.kvip_hip_fetch_gather(ctypes.byref(fetch), None) == abi.KVIP_ERR_INVALID


def test_resident_entry_points_reject_before_launch():
    lib = abi.load_library()
    for name in ("kvip_hip_resident_round", "kvip_hip_resident_begin", "kvip_hip_resident_finish",
                 "kvip_hip_resident_prepare"):
        assert getattr(lib, name)(None, None) == abi.KVIP_ERR_INVALID, name
    assert lib.kvip_hip_resident_prefetch(None, None, None) == abi.KVIP_ERR_INVALID
    assert lib.kvip_hip_resident_score(None, None, None, None) == abi.KVIP_ERR_INVALID
    # Well-formed resident arguments, then a prefetch whose windows do not fit the cold range
    # and one half of the prefetch records missing.
    names = [f for f, _ in abi.ResidentArgs._fields_]
    ptrs = {n: 256 for n in names[:21]}
    args = abi.ResidentArgs(**ptrs, host_pool_bytes=1 << 20, batch=1, rows_per_request=1, owners=1, history=8192,
                            resident=4096, hot_stride=4096, row_bytes=656, used=0, prefetch_tokens=256,
                            prefetch_counts=256)
    pf = abi.PrefetchArgs(victim_hits=256, cold_hits=256, cold_words=128, windows=32, window_limit=64,
                          prefetch_limit=512)
    assert lib.kvip_hip_resident_prefetch(ctypes.byref(args), ctypes.byref(pf), None) == abi.KVIP_ERR_INVALID
    pf.windows, pf.window_limit = 4, 481
    assert lib.kvip_hip_resident_prefetch(ctypes.byref(args), ctypes.byref(pf), None) == abi.KVIP_ERR_INVALID
    args.prefetch_counts = 0
    assert lib.kvip_hip_resident_begin(ctypes.byref(args), None) == abi.KVIP_ERR_INVALID
    # ABC tail bounds need at least 384 ring slots after the hot ones.
    args.prefetch_counts, args.tail_bounds, args.hot_stride = 256, 256, 4096 + 256
    assert lib.kvip_hip_resident_begin(ctypes.byref(args), None) == abi.KVIP_ERR_INVALID


def test_lidu_arguments_rejected_before_launch():
    lib = abi.load_library()
    assert lib.kvip_hip_lidu(None, None) == abi.KVIP_ERR_INVALID
    assert lib.kvip_hip_lidu_workspace_bytes(0) == 0
    need = lib.kvip_hip_lidu_workspace_bytes(2)
    assert need >= 2 * (3 * 8192 + 16) * 4
    names = [f for f, _ in abi.LiduArgs._fields_ if f not in ("profiling", "workspace_bytes")][:20]
    good = dict({n: 256 for n in names}, workspace_bytes=need, batch=2, packed_queries=8, pool_size=2,
                source_capacity=4096, resident_capacity=4096, resident_blocks=32, layer_id=0, num_layers=1,
                max_num_reqs=2, qcap=32)
    bad_cases = [dict(batch=0), dict(packed_queries=9), dict(packed_queries=1), dict(resident_capacity=2047),
                 dict(source_capacity=(1 << 20) + 20 * 128 + 1), dict(layer_id=1), dict(max_num_reqs=1),
                 dict(workspace_bytes=need - 1), dict(topk=260), dict(destination_slots=264),
                 dict(qcap=1 << 30, num_layers=1, max_num_reqs=4), dict(topk=0)]
    for case in bad_cases:
        args = abi.LiduArgs(**dict(good, **case))
        assert lib.kvip_hip_lidu(ctypes.byref(args), None) == abi.KVIP_ERR_INVALID, case


def test_binding_validation_cpu():
    torch = pytest.importorskip("torch")
    from kvip_amd.operators.lifetch.binding import LIFetchBinding

    with pytest.raises(ValueError):
        LIFetchBinding(torch, batch=0, max_context=4096, device="cpu")
    with pytest.raises(ValueError):
        LIFetchBinding(torch, batch=1, max_context=4096, device="cpu", heads=16)
    rot = LIFetchBinding(torch, batch=2, max_context=1000, device="cpu")
    assert rot.max_blocks == 8 and rot.key_stride == 1024
    with pytest.raises(ValueError):
        rot.bind_index_cache(torch.zeros((4, 128, 128), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        rot.indexer_args()


def test_forward_set_options_cpu():
    """LIFetch.set_options keeps the reference's keyword-only call
    (python/kvip/operators/lifetch/streaming.py:133): construction applies the defaults,
    deferred_fetch is recorded, diagnostics=True (in-kernel cycle stamps) and non-bool
    values are refused; nothing is launched."""
    torch = pytest.importorskip("torch")
    import kvip_amd

    rot = kvip_amd.LIFetchBinding(torch, batch=2, max_context=4096, device="cpu")
    rot.bind_index_cache(torch.zeros((rot.batch * rot.max_blocks, 128, 128), dtype=torch.float8_e4m3fn))
    upd = kvip_amd.ContiguousFetch(torch, rot, torch.zeros((rot.batch * rot.max_blocks, 128, 656), dtype=torch.uint8))
    fwd = kvip_amd.LIFetch(rot, upd)
    assert (fwd.diagnostics, fwd.deferred_fetch) == (False, False)
    fwd.set_options(deferred_fetch=True)
    assert fwd.deferred_fetch is True
    fwd.set_options()
    assert fwd.deferred_fetch is False
    with pytest.raises(ValueError):
        fwd.set_options(diagnostics=True)
    with pytest.raises(ValueError):
        fwd.set_options(deferred_fetch=1)
    with pytest.raises(TypeError):
        fwd.set_options(True)
    assert fwd.plan == "three"


def test_lifetch_plan_query():
    """kvip_hip_lifetch_plan picks the forward's launch plan from the arguments alone."""
    lib = abi.load_library()
    assert lib.kvip_hip_lifetch_plan(None) == abi.KVIP_ERR_INVALID

    def make(**over):
        o = dict(qk=abi.DTYPE_FP8_E4M3, rpr=1, batch=64, segments=0x8000, histogram=0x7000)
        o.update(over)
        li = abi.IndexerArgs(query=0x1000, weights=0x1100, keys=0x2000, block_table=0x3000, seq_lens=0x4000,
                             score_keys=0x5000, histogram=o["histogram"], key_block_stride=128 * 128 * 2, batch=o["batch"],
                             rows_per_request=o["rpr"], heads=64, max_blocks=256, num_blocks=1024,
                             key_stride=32768, qk_dtype=o["qk"], weight_dtype=abi.DTYPE_FP32)
        tk = abi.TopkArgs(score_keys=0x5000, histogram=o["histogram"], segments=o["segments"], seq_lens=0x4000,
                          topk=0x6000, batch=o["batch"], rows_per_request=o["rpr"], key_stride=32768)
        fe = abi.FetchArgs(topk=0x6000, kv_cache=0xA000, block_table=0x3000, output=0xB000,
                           kv_block_stride=128 * 656, row_stride=656, row_bytes=656, batch=o["batch"],
                           rows_per_request=o["rpr"], max_blocks=256, num_blocks=1024)
        return abi.LIFetchArgs(li, tk, fe)

    plan = lambda a: abi.LIFETCH_PLANS.get(lib.kvip_hip_lifetch_plan(ctypes.byref(a)), "invalid")  # noqa: E731
    assert plan(make()) == "three"
    assert plan(make(segments=0)) == "three"
    assert plan(make(qk=abi.DTYPE_BF16)) == "three"
    assert plan(make(rpr=2)) == "three"
    assert plan(make(histogram=0)) == "invalid"                 # decode scoring always fills a histogram
    bad = make()
    bad.fetch.topk = 0x6100                                     # stages not chained
    assert plan(bad) == "invalid"
