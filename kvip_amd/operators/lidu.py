"""`kvip_amd.lidu`: the LIDU batch transaction on the device.

Same call as the reference's ``kvip.lidu`` (python/kvip/operators/lidu.py:4-8), which is
the out-variant op ``lidu_fused_batch_get_prepare_mtp_out``
(csrc/operators/lidu/torch_extension/csrc/lidu_fused_batch_get_prepare_mtp_ops.cpp:195-270):
20 tensors and four integers in the reference's order, the six outputs returned. The
tensor checks mirror the reference host op (:41-190) and raise ValueError. The work is
enqueued on torch's current stream of the tensors' device through ``kvip_hip_lidu``
(libkvip_hip.so); the per-batch workspace is allocated once per (device, batch) and
reused, so the call can be captured in a CUDA graph after a first eager call.

`lidu_prepare` is the allocating variant ``lidu_fused_batch_get_prepare_mtp`` (:272-300).
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi

SPARSE = 2048
MAX_QUERIES = 4
MISS_CAPACITY = SPARSE * MAX_QUERIES
MISS_SLOT_BITMAP_WORDS = 4176
MAX_SOURCE_CAPACITY = (1 << 20) + 20 * 128
PROFILE_LANES = 8
PROFILE_FIELDS = 32
INT32_MAX = (1 << 31) - 1

_WORKSPACES = {}


def _torch():
    import torch

    return torch


def _workspace(torch, lib, device, batch):
    key = (str(device), batch)
    ws = _WORKSPACES.get(key)
    if ws is None:
        nbytes = int(lib.kvip_hip_lidu_workspace_bytes(batch))
        ws = torch.empty(nbytes // 4, dtype=torch.int32, device=device)
        _WORKSPACES[key] = ws
    return ws


def _check_inputs(torch, topk, query_ends, pool_entries, t2s, s2t, cursors, cache_tokens, candidate_lens,
                  miss_slots, miss_slot_bitmap, block_table, logical, profile_enabled, layer_id, num_layers,
                  max_num_reqs, qcap):
    if topk.dim() != 3 or topk.shape[0] < 1 or topk.shape[1] != 1 or topk.shape[2] != SPARSE:
        raise ValueError("lidu: topk_indices must be int32 [T,1,2048]")
    if query_ends.dim() != 1 or query_ends.shape[0] < 1:
        raise ValueError("lidu: actual_seq_lengths_query must be int32 [B]")
    batch, packed = query_ends.shape[0], topk.shape[0]
    if not batch <= packed <= MAX_QUERIES * batch:
        raise ValueError("lidu: requires 1--4 packed queries per request")
    for name, t in (("req_pool_entries", pool_entries), ("cache_tokens", cache_tokens),
                    ("candidate_lens", candidate_lens), ("logical_seq_lengths", logical)):
        if t.dim() != 1 or t.shape[0] != batch:
            raise ValueError(f"lidu: {name} must be int32 [B]")
    if profile_enabled.dim() != 1 or profile_enabled.shape[0] != 1:
        raise ValueError("lidu: profile_enabled must be int32 [1]")
    if tuple(miss_slots.shape) != (batch, SPARSE):
        raise ValueError("lidu: miss_slots must be int32 [B,2048]")
    if tuple(miss_slot_bitmap.shape) != (batch, MISS_SLOT_BITMAP_WORDS):
        raise ValueError(f"lidu: miss_slot_bitmap must be int32 [B,{MISS_SLOT_BITMAP_WORDS}]")
    if t2s.dim() != 2 or t2s.shape[0] < 1 or not 0 < t2s.shape[1] <= MAX_SOURCE_CAPACITY:
        raise ValueError("lidu: token_to_slot_pool must be [pool,source_capacity]")
    if s2t.dim() != 2 or s2t.shape[0] != t2s.shape[0] or s2t.shape[1] < SPARSE:
        raise ValueError("lidu: slot_to_token_pool must be [pool,resident_capacity >= 2048]")
    if cursors.dim() != 1 or cursors.shape[0] != t2s.shape[0]:
        raise ValueError("lidu: eviction_cursors must be int32 [pool]")
    if block_table.dim() != 2 or block_table.shape[0] != batch or block_table.shape[1] < 1:
        raise ValueError("lidu: resident_block_table must be int32 [B,resident_blocks]")
    if not (0 <= layer_id < num_layers and max_num_reqs >= batch and qcap > 0
            and max_num_reqs * num_layers * qcap <= INT32_MAX and block_table.shape[1] * 128 <= INT32_MAX):
        raise ValueError("lidu: AccessTable geometry is invalid")
    tensors = (topk, query_ends, pool_entries, t2s, s2t, cursors, cache_tokens, candidate_lens, miss_slots,
               miss_slot_bitmap, block_table, logical, profile_enabled)
    for t in tensors:
        if t.dtype != torch.int32:
            raise ValueError("lidu: supports only int32 inputs")
        if t.device != topk.device or not t.is_contiguous():
            raise ValueError("lidu: tensors must be contiguous and on one GPU")
    if topk.device.type != "cuda":
        raise ValueError("lidu: inputs must be GPU tensors (kvip_amd has no CPU path)")
    return batch, packed


def _check_outputs(torch, topk, batch, dest, counts, indices, offsets, output_indices, resident, profiling):
    if tuple(dest.shape) != tuple(topk.shape):
        raise ValueError("lidu: destination_slots must be int32 [T,1,2048]")
    cap = batch * MISS_CAPACITY
    if (counts.dim() != 1 or counts.shape[0] != batch + 1 or indices.dim() != 1 or indices.numel() != cap
            or offsets.dim() != 1 or offsets.numel() != cap or output_indices.dim() != 1
            or output_indices.numel() != cap or resident.dim() != 1 or resident.shape[0] != batch):
        raise ValueError("lidu: descriptors must be int32 [B*8192], with miss_counts int32 [B+1] and "
                         "resident_seq_lengths int32 [B]")
    for t in (dest, counts, indices, offsets, output_indices, resident):
        if t.dtype != torch.int32 or t.device != topk.device or not t.is_contiguous():
            raise ValueError("lidu: outputs must be contiguous int32 tensors on the input GPU")
    if (tuple(profiling.shape) != (batch, PROFILE_LANES, PROFILE_FIELDS) or profiling.dtype != torch.int64
            or profiling.device != topk.device or not profiling.is_contiguous()):
        raise ValueError("lidu: profiling must be contiguous int64 [B,8,32] on the input GPU")


def lidu(topk_indices, actual_seq_lengths_query, req_pool_entries, token_to_slot_pool, slot_to_token_pool,
         eviction_cursors, cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table,
         logical_seq_lengths, profile_enabled, destination_slots, miss_counts, indices, offsets, output_indices,
         resident_seq_lengths, profiling, layer_id, num_layers, max_num_reqs, qcap):
    """Run the LIDU transaction; token_to_slot_pool, slot_to_token_pool, eviction_cursors and the
    outputs are written in place. Returns (destination_slots, miss_counts, indices, offsets,
    output_indices, resident_seq_lengths)."""
    torch = _torch()
    batch, packed = _check_inputs(
        torch, topk_indices, actual_seq_lengths_query, req_pool_entries, token_to_slot_pool, slot_to_token_pool,
        eviction_cursors, cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table,
        logical_seq_lengths, profile_enabled, layer_id, num_layers, max_num_reqs, qcap)
    _check_outputs(torch, topk_indices, batch, destination_slots, miss_counts, indices, offsets, output_indices,
                   resident_seq_lengths, profiling)
    lib = abi.load_library()
    device = abi.device_of(torch, topk_indices.device)
    ws = _workspace(torch, lib, device, batch)
    p = abi.ptr
    args = abi.LiduArgs(
        topk=p(topk_indices), actual_seq_lengths_query=p(actual_seq_lengths_query),
        req_pool_entries=p(req_pool_entries), token_to_slot=p(token_to_slot_pool),
        slot_to_token=p(slot_to_token_pool), eviction_cursors=p(eviction_cursors), cache_tokens=p(cache_tokens),
        candidate_lens=p(candidate_lens), miss_slots=p(miss_slots), miss_slot_bitmap=p(miss_slot_bitmap),
        resident_block_table=p(resident_block_table), logical_seq_lengths=p(logical_seq_lengths),
        profile_enabled=p(profile_enabled), destination_slots=p(destination_slots), miss_counts=p(miss_counts),
        indices=p(indices), offsets=p(offsets), output_indices=p(output_indices),
        resident_seq_lengths=p(resident_seq_lengths), profiling=p(profiling), workspace=p(ws),
        workspace_bytes=ws.numel() * 4, batch=batch, packed_queries=packed, pool_size=token_to_slot_pool.shape[0],
        source_capacity=token_to_slot_pool.shape[1], resident_capacity=slot_to_token_pool.shape[1],
        resident_blocks=resident_block_table.shape[1], layer_id=layer_id, num_layers=num_layers,
        max_num_reqs=max_num_reqs, qcap=qcap,
    )
    abi.check(lib.kvip_hip_lidu(ctypes.byref(args), abi.stream_handle(torch, device)), "lidu")
    return destination_slots, miss_counts, indices, offsets, output_indices, resident_seq_lengths


def lidu_prepare(topk_indices, actual_seq_lengths_query, req_pool_entries, token_to_slot_pool, slot_to_token_pool,
                 eviction_cursors, cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table,
                 logical_seq_lengths, profile_enabled, layer_id, num_layers, max_num_reqs, qcap):
    """Allocating variant: returns fresh (destination_slots, miss_counts, indices, offsets,
    output_indices, resident_seq_lengths)."""
    torch = _torch()
    dev = topk_indices.device
    batch = actual_seq_lengths_query.shape[0]
    cap = batch * MISS_CAPACITY
    outs = (torch.empty(topk_indices.shape, dtype=torch.int32, device=dev),
            torch.empty(batch + 1, dtype=torch.int32, device=dev),
            torch.empty(cap, dtype=torch.int32, device=dev), torch.empty(cap, dtype=torch.int32, device=dev),
            torch.empty(cap, dtype=torch.int32, device=dev), torch.empty(batch, dtype=torch.int32, device=dev))
    profiling = torch.zeros((batch, PROFILE_LANES, PROFILE_FIELDS), dtype=torch.int64, device=dev)
    return lidu(topk_indices, actual_seq_lengths_query, req_pool_entries, token_to_slot_pool, slot_to_token_pool,
                eviction_cursors, cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table,
                logical_seq_lengths, profile_enabled, *outs, profiling, layer_id, num_layers, max_num_reqs, qcap)
