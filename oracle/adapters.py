"""CPU restatement of the vLLM adapter's device work (decode query packing and Index-K
ingestion). TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

prepare_metadata - QueryInputs.prepare (python/kvip/adapters/vllm/inputs.py:75-125)
bind_positions   - QueryInputs.bind_positions (:127-133)
pack             - QueryInputs.pack (:135-152), a byte gather
ingest_decode    - VllmIndexCacheStorage.ingest_decode (adapters/vllm/index_import.py:39-52)
ingest_prefill   - VllmIndexCacheStorage.ingest_prefill (:18-37)
publish_outputs  - token-order (TND) publication of the Index update's outputs
                   (operators/lifetch/index_update.py:18-21; op_kernel/streaming.cpp:31-44,
                   :66-89); pinned by the inverse-of-gather property in
                   tests/test_oracle_adapters.py
Pinned by the known answers of tests/adapters/test_inputs.py (tests/test_oracle_adapters.py).
"""
from __future__ import annotations

import numpy as np

Q = 4


def prepare_metadata(batch, counts, starts=None, owners=None):
    """int64 [5, batch*4]: gather indices, query validity, unpack indices, output
    validity, row owners (int32 pairs packed in the last row)."""
    meta = np.zeros((5, batch * Q), np.int64)
    owner_words = meta[4].view(np.int32)
    if owners is not None:
        owner_words[:len(owners)] = owners
    begin = 0
    for row, count in enumerate(counts):
        slot = row * Q
        source = begin if starts is None else starts[row]
        for k in range(count):
            meta[0, slot + k] = source + k
            meta[1, slot + k] = 1
            meta[2, begin + k] = slot + k
            meta[3, begin + k] = 1
        begin += count
    return meta


def bind_positions(meta, positions):
    ends = (positions[meta[0]] + 1) * meta[1]
    return ends.astype(np.int32)


def pack(meta, query, weights, scale):
    """query uint8 [tokens, H, 128], weights [tokens, H], scale [tokens, H]."""
    g = meta[0]
    return query[g], weights[g], scale[g]


def ingest_decode(keys, scales, source_keys, source_scales, slot_mapping, meta, query_ends, owners, history):
    """keys uint8 [owners, history, 128], scales f32 [owners, history]; in place."""
    flat_k = keys.reshape(-1, 128)
    flat_s = scales.reshape(-1)
    rows = query_ends.size
    for r in range(rows):
        valid = query_ends[r] > 0
        src = int(slot_mapping[meta[0, r]]) if valid else 0
        dst = int(owners[r // Q]) * history + int(query_ends[r]) - 1 if valid else r
        flat_k[dst] = source_keys[src]
        flat_s[dst] = source_scales[src]


def ingest_prefill(keys, scales, source_keys, source_scales, block_table, block_size, slot_mapping, plans,
                   positions, imported):
    """plans: (owner, start, begin, stop) per row; `imported` is the set of owners already
    imported (updated). In place."""
    for row, (owner, start, begin, stop) in enumerate(plans):
        if owner not in imported and start:
            for t in range(start):
                src = int(block_table[row][t // block_size]) * block_size + t % block_size
                keys[owner, t] = source_keys[src]
                scales[owner, t] = source_scales[src]
        imported.add(owner)
        for j in range(begin, stop):
            keys[owner, positions[j]] = source_keys[slot_mapping[j]]
            scales[owner, positions[j]] = source_scales[slot_mapping[j]]


def publish_outputs(meta, rows):
    """rows [batch*4, ...] in query-row (slot) order -> token order: output row t holds
    query row unpack[t] when output_valid[t], else -1 throughout."""
    out = np.full_like(rows, -1)
    for t in range(meta.shape[1]):
        if meta[3, t]:
            out[t] = rows[int(meta[2, t])]
    return out
