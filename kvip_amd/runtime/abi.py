"""ctypes view of include/kvip_hip.h and the loader of libkvip_hip.so.

The library is the only compute path: there is no CPU or PyTorch fallback. Loading
fails loudly when the in-tree library is missing or was built for another ABI.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parents[1] / "_lib" / "libkvip_hip.so"
ABI_VERSION = 15

KVIP_OK = 0
KVIP_ERR_INVALID = 100000

DTYPE_FP8_E4M3 = 0
DTYPE_BF16 = 1
DTYPE_FP32 = 2

STATUS_BAD_BLOCK = 1
STATUS_HISTOGRAM = 2
STATUS_BAD_TOKEN = 4

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class IndexerArgs(ctypes.Structure):
    _fields_ = [
        ("query", _p), ("weights", _p), ("query_scale", _p), ("keys", _p), ("key_scale", _p),
        ("block_table", _p), ("seq_lens", _p), ("query_ends", _p), ("score_keys", _p),
        ("histogram", _p), ("status", _p),
        ("key_block_stride", _i64), ("scale_block_stride", _i64),
        ("batch", _i32), ("rows_per_request", _i32), ("heads", _i32), ("max_blocks", _i32),
        ("num_blocks", _i32), ("key_stride", _i32), ("qk_dtype", _i32), ("weight_dtype", _i32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("query", _p), ("weights", _p), ("query_scale", _p), ("keys", _p), ("key_scale", _p), ("block_table", _p),
        ("cu_seqlens_q", _p), ("seq_lens_k", _p), ("score_keys", _p), ("histogram", _p), ("row_valid", _p),
        ("status", _p),
        ("key_block_stride", _i64), ("scale_block_stride", _i64),
        ("sequences", _i32), ("rows", _i32), ("heads", _i32), ("max_blocks", _i32), ("num_blocks", _i32),
        ("key_stride", _i32), ("qk_dtype", _i32), ("weight_dtype", _i32),
    ]


class TopkArgs(ctypes.Structure):
    _fields_ = [
        ("score_keys", _p), ("histogram", _p), ("segments", _p), ("seq_lens", _p), ("query_ends", _p), ("topk", _p),
        ("status", _p),
        ("batch", _i32), ("rows_per_request", _i32), ("key_stride", _i32), ("limit", _i32),
    ]


class FetchArgs(ctypes.Structure):
    _fields_ = [
        ("topk", _p), ("kv_cache", _p), ("block_table", _p), ("output", _p), ("status", _p),
        ("kv_block_stride", _i64),
        ("row_stride", _i32), ("row_bytes", _i32), ("batch", _i32), ("rows_per_request", _i32),
        ("max_blocks", _i32), ("num_blocks", _i32),
    ]


class LIFetchArgs(ctypes.Structure):
    _fields_ = [("indexer", IndexerArgs), ("topk", TopkArgs), ("fetch", FetchArgs)]


class AbcArgs(ctypes.Structure):
    _fields_ = [
        ("token_to_slot", _p), ("slot_to_token", _p), ("descriptors", _p), ("status", _p),
        ("groups", _i32), ("rows", _i32), ("requests", _i32), ("layers", _i32), ("pool", _i32),
        ("t2s_tokens", _i32), ("s2t_tokens", _i32), ("history", _i32), ("tail", _i32),
    ]


class LruArgs(ctypes.Structure):
    _fields_ = [
        ("order", _p), ("scratch", _p), ("slots", _p), ("bitmap", _p),
        ("capacity", _i32), ("bitmap_words", _i32),
    ]


class LiduArgs(ctypes.Structure):
    _fields_ = [
        ("topk", _p), ("actual_seq_lengths_query", _p), ("req_pool_entries", _p), ("token_to_slot", _p),
        ("slot_to_token", _p), ("eviction_cursors", _p), ("cache_tokens", _p), ("candidate_lens", _p),
        ("miss_slots", _p), ("miss_slot_bitmap", _p), ("resident_block_table", _p), ("logical_seq_lengths", _p),
        ("profile_enabled", _p), ("destination_slots", _p), ("miss_counts", _p), ("indices", _p),
        ("offsets", _p), ("output_indices", _p), ("resident_seq_lengths", _p), ("profiling", _p),
        ("workspace", _p), ("workspace_bytes", _i64),
        ("batch", _i32), ("packed_queries", _i32), ("pool_size", _i32), ("source_capacity", _i32),
        ("resident_capacity", _i32), ("resident_blocks", _i32), ("layer_id", _i32), ("num_layers", _i32),
        ("max_num_reqs", _i32), ("qcap", _i32),
    ]


class QueryPackArgs(ctypes.Structure):
    _fields_ = [
        ("gather_indices", _p), ("query_valid", _p), ("positions", _p), ("query_ends", _p), ("query_in", _p),
        ("weights_in", _p), ("scale_in", _p), ("query_out", _p), ("weights_out", _p), ("scale_out", _p),
        ("status", _p), ("tokens", _i64), ("rows", _i32), ("heads", _i32),
    ]


# kvip_hip_lifetch_plan results.
LIFETCH_PLANS = {0: "three"}
TOPK_REGS_MAX_KEYS = 65536  # KVIP_TOPK_REGS_MAX_KEYS
LIFETCH_STATIC_SCRATCH_BYTES = 16 << 20  # KVIP_LIFETCH_STATIC_SCRATCH_BYTES

INGEST_DECODE = 0
INGEST_LIST = 1
INGEST_PREFIX = 2


class IngestArgs(ctypes.Structure):
    _fields_ = [
        ("source_keys", _p), ("source_scales", _p), ("target_keys", _p), ("target_scales", _p),
        ("query_ends", _p), ("gather_indices", _p), ("slot_mapping", _p), ("row_owners", _p),
        ("sources", _p), ("targets", _p), ("block_table", _p), ("status", _p),
        ("source_rows", _i64), ("target_rows", _i64), ("count", _i64), ("history", _i64), ("target_base", _i64),
        ("slot_count", _i64), ("mode", _i32), ("queries_per_request", _i32), ("block_size", _i32),
        ("reserved", _i32),
    ]


RESIDENT_MAX_QUERIES = 4
RESIDENT_MAX_RESIDENT = 131072
RESIDENT_LRU_SLOTS = 2048
RESIDENT_ERR_TOKEN = 1
RESIDENT_ERR_CANDIDATE = 4
RESIDENT_ERR_SOURCE = 8
RESIDENT_ERR_UPDATE = 16


class ResidentArgs(ctypes.Structure):
    _fields_ = [
        ("topk", _p), ("row_owners", _p), ("lru_slots", _p), ("reserved_hot", _p), ("hot_valid", _p),
        ("index_keys", _p), ("index_scales", _p), ("addresses", _p), ("logical_ids", _p), ("host_pool", _p),
        ("hot_cache", _p), ("logical_output", _p), ("slot_output", _p), ("changes", _p), ("change_slots", _p),
        ("miss_counts", _p), ("fetch_sources", _p), ("fetch_slots", _p), ("fetch_positions", _p), ("status", _p),
        ("workspace", _p), ("host_pool_bytes", _i64),
        ("batch", _i32), ("rows_per_request", _i32), ("owners", _i32), ("history", _i32), ("resident", _i32),
        ("hot_stride", _i32), ("row_bytes", _i32), ("used", _i32), ("unpack_indices", _p), ("output_valid", _p),
        ("tail_bounds", _p), ("prefetch_tokens", _p), ("prefetch_counts", _p),
    ]


class PrefixClassifyArgs(ctypes.Structure):
    _fields_ = [
        ("score_keys", _p), ("prefix_topk", _p), ("seq_lens", _p), ("query_ends", _p), ("lru_slots", _p),
        ("thresholds", _p), ("victim_hits", _p), ("cold_hits", _p),
        ("batch", _i32), ("rows_per_request", _i32), ("key_stride", _i32), ("resident", _i32), ("cold_words", _i32),
        ("reserved", _i32),
    ]


PREFETCH_MAX_WINDOWS = 32  # KVIP_PREFETCH_MAX_WINDOWS


class PrefetchArgs(ctypes.Structure):
    _fields_ = [
        ("victim_hits", _p), ("cold_hits", _p), ("window_counts", _p), ("cold_words", _i32), ("windows", _i32),
        ("window_limit", _i32), ("prefetch_limit", _i32),
    ]


class PageArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _p), ("addresses", _p), ("valid", _p), ("token_to_slot", _p), ("fused", _p), ("status", _p),
        ("entries", _i64), ("map_entries", _i64), ("count", _i32), ("groups", _i32), ("pages", _i32),
        ("block_size", _i32), ("history", _i32), ("reserved", _i32),
    ]


class SparseAttnArgs(ctypes.Structure):
    _fields_ = [
        ("query", _p), ("kv_cache", _p), ("block_table", _p), ("indices", _p), ("output", _p), ("status", _p),
        ("workspace", _p), ("kv_block_stride", _i64), ("row_stride", _i32), ("rows", _i32), ("rows_per_request", _i32),
        ("heads", _i32), ("max_blocks", _i32), ("num_blocks", _i32), ("scale", ctypes.c_float), ("reserved", _i32),
    ]


# name -> (argtypes, restype); must list every function declared in include/kvip_hip.h.
PROTOTYPES = {
    "kvip_hip_abi_version": ([], ctypes.c_uint32),
    "kvip_hip_sparse_attention": ([ctypes.POINTER(SparseAttnArgs), _p], ctypes.c_uint32),
    "kvip_hip_sparse_attention_workspace_bytes": ([_i32, _i32], ctypes.c_uint64),
    "kvip_hip_publish_pages": ([ctypes.POINTER(PageArgs), _p], ctypes.c_uint32),
    "kvip_hip_indexer_decode": ([ctypes.POINTER(IndexerArgs), _p], ctypes.c_uint32),
    "kvip_hip_indexer_decode_window": ([ctypes.POINTER(IndexerArgs), _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_indexer_prefill": ([ctypes.POINTER(PrefillArgs), _p], ctypes.c_uint32),
    "kvip_hip_indexer_prefill_grid": ([ctypes.POINTER(PrefillArgs), ctypes.c_int32, _p], ctypes.c_uint32),
    "kvip_hip_topk": ([ctypes.POINTER(TopkArgs), _p], ctypes.c_uint32),
    "kvip_hip_fetch_gather": ([ctypes.POINTER(FetchArgs), _p], ctypes.c_uint32),
    "kvip_hip_lifetch_forward": ([ctypes.POINTER(LIFetchArgs), _p], ctypes.c_uint32),
    "kvip_hip_lifetch_plan": ([ctypes.POINTER(LIFetchArgs)], ctypes.c_uint32),
    "kvip_hip_lifetch_forward_static": ([ctypes.POINTER(LIFetchArgs), _p], ctypes.c_uint32),
    "kvip_hip_select_fetch": ([ctypes.POINTER(TopkArgs), ctypes.POINTER(FetchArgs), _p], ctypes.c_uint32),
    "kvip_hip_update_abc": ([ctypes.POINTER(AbcArgs), _p], ctypes.c_uint32),
    "kvip_hip_lru_reset": ([ctypes.POINTER(LruArgs), _i32, _p], ctypes.c_uint32),
    "kvip_hip_lru_extend": ([ctypes.POINTER(LruArgs), _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_lru_commit": ([ctypes.POINTER(LruArgs), _p, _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_lru_reset_chains": ([ctypes.POINTER(LruArgs), _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_lru_commit_chains": ([ctypes.POINTER(LruArgs), _i32, _p, ctypes.c_int64, _i32, _i32, _p],
                                   ctypes.c_uint32),
    "kvip_hip_lidu_workspace_bytes": ([_i32], ctypes.c_uint64),
    "kvip_hip_lidu": ([ctypes.POINTER(LiduArgs), _p], ctypes.c_uint32),
    "kvip_hip_pack_queries": ([ctypes.POINTER(QueryPackArgs), _p], ctypes.c_uint32),
    "kvip_hip_ingest_index": ([ctypes.POINTER(IngestArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_prefix": ([ctypes.POINTER(TopkArgs), ctypes.POINTER(PrefixClassifyArgs), _p],
                                 ctypes.c_uint32),
    "kvip_hip_resident_workspace_bytes": ([_i32, _i32], ctypes.c_uint64),
    "kvip_hip_resident_prepare": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_round": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_begin": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_finish": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_resolve": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_fetch": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_update": ([ctypes.POINTER(ResidentArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_prefetch": ([ctypes.POINTER(ResidentArgs), ctypes.POINTER(PrefetchArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_prefetch_windows": ([ctypes.POINTER(ResidentArgs), ctypes.POINTER(PrefetchArgs), _i32, _i32, _p],
                                           ctypes.c_uint32),
    "kvip_hip_resident_prefetch_copy": ([ctypes.POINTER(ResidentArgs), ctypes.POINTER(PrefetchArgs), _i32, _i32, _p],
                                        ctypes.c_uint32),
    "kvip_hip_resident_threshold": ([ctypes.POINTER(TopkArgs), ctypes.POINTER(PrefixClassifyArgs), _p], ctypes.c_uint32),
    "kvip_hip_resident_cold_hits": ([ctypes.POINTER(PrefixClassifyArgs), _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_resident_score_window": ([ctypes.POINTER(IndexerArgs), ctypes.POINTER(TopkArgs),
                                        ctypes.POINTER(ResidentArgs), _i32, _i32, _p], ctypes.c_uint32),
    "kvip_hip_resident_score": ([ctypes.POINTER(IndexerArgs), ctypes.POINTER(TopkArgs), ctypes.POINTER(ResidentArgs),
                                 _p], ctypes.c_uint32),
    "kvip_hip_resident_forward": ([ctypes.POINTER(IndexerArgs), ctypes.POINTER(TopkArgs), ctypes.POINTER(ResidentArgs),
                                   _p], ctypes.c_uint32),
}

_LIB = None


def load_library(path: Path | None = None):
    """Load libkvip_hip.so once and bind the prototypes. Raises RuntimeError if the
    library is missing or its ABI version differs."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    path = Path(path) if path is not None else LIBRARY
    # torch ships its own libamdhip64 (same soname): load it first so that the library
    # binds to the one HIP runtime that owns torch's streams and allocations.
    import torch  # noqa: F401

    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(kvip_amd has no CPU fallback)"
        )
    lib = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = argtypes, restype
    version = lib.kvip_hip_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libkvip_hip.so ABI {version} != expected {ABI_VERSION}; rebuild")
    if path == LIBRARY:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == KVIP_ERR_INVALID:
        raise ValueError(f"{what}: arguments rejected by libkvip_hip")
    if rc != KVIP_OK:
        raise RuntimeError(f"{what}: HIP launch failed with hipError {rc}")


def ptr(tensor) -> int:
    """Device address of a tensor, or 0 for None."""
    return 0 if tensor is None else int(tensor.data_ptr())


def device_of(torch, device):
    """torch.device with an explicit index ("cuda" -> "cuda:<current>")."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


def stream_handle(torch, device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)
