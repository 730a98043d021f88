"""MI355X-native lightning-indexer-with-fetch (KVIP's LIFetch path) on gfx950.

Public names are resolved lazily, as in the reference package
(python/kvip/__init__.py:18-43). Every compute call goes through libkvip_hip.so;
there is no CPU fallback.
"""
from importlib import import_module

__all__ = [
    "QueryInputs",
    "IndexCacheStorage",
    "LIFetch",
    "LIFetchBinding",
    "ContiguousFetch",
    "ResidentIndexUpdate",
    "ResidentPrefix",
    "ResidentPrefetch",
    "PrefillIndexer",
    "quant_lightning_indexer",
    "MixedRound",
    "SparseAttention",
    "sparse_attention",
    "VllmIndexSelector",
    "PagedIndexer",
    "RequestPlan",
    "SlotLRU",
    "SlotLRUChains",
    "PageUpdates",
    "update_abc",
    "lidu",
    "lidu_prepare",
    "lidu_reserve",
    "register_torch_ops",
    "build_libraries",
    "load_library",
]

_EXPORTS = {
    "QueryInputs": ("adapters.vllm.inputs", "QueryInputs"),
    "IndexCacheStorage": ("adapters.vllm.index_import", "VllmIndexCacheStorage"),
    "LIFetch": ("operators.lifetch.forward", "LIFetchForward"),
    "LIFetchBinding": ("operators.lifetch.binding", "LIFetchBinding"),
    "ContiguousFetch": ("operators.lifetch.binding", "ContiguousFetch"),
    "ResidentIndexUpdate": ("operators.lifetch.resident", "ResidentIndexUpdate"),
    "ResidentPrefix": ("operators.lifetch.resident", "ResidentPrefix"),
    "ResidentPrefetch": ("operators.lifetch.resident", "ResidentPrefetch"),
    "PrefillIndexer": ("operators.prefill", "PrefillIndexer"),
    "quant_lightning_indexer": ("operators.prefill", "quant_lightning_indexer"),
    "MixedRound": ("operators.mixed", "MixedRound"),
    "SparseAttention": ("operators.sfa", "SparseAttention"),
    "sparse_attention": ("operators.sfa", "sparse_attention"),
    "VllmIndexSelector": ("adapters.vllm.selector", "VllmIndexSelector"),
    "PagedIndexer": ("adapters.vllm.selector", "PagedIndexer"),
    "RequestPlan": ("adapters.vllm.selector", "RequestPlan"),
    "SlotLRU": ("cache.lru", "SlotLRU"),
    "SlotLRUChains": ("cache.lru", "SlotLRUChains"),
    "PageUpdates": ("cache.page_updates", "PageUpdates"),
    "update_abc": ("cache.abc", "update_abc"),
    "lidu": ("operators.lidu", "lidu"),
    "lidu_prepare": ("operators.lidu", "lidu_prepare"),
    "lidu_reserve": ("operators.lidu", "lidu_reserve"),
    "register_torch_ops": ("operators.lidu", "register_torch_ops"),
    "build_libraries": ("runtime.build", "build_libraries"),
    "load_library": ("runtime.abi", "load_library"),
}


def __getattr__(name):
    if name not in _EXPORTS:
        raise AttributeError(name)
    module, symbol = _EXPORTS[name]
    return getattr(import_module(f"{__name__}.{module}"), symbol)
