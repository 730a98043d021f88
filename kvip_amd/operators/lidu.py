"""`kvip_amd.lidu`: the LIDU batch transaction on the device.

Same call as the reference's ``kvip.lidu`` (python/kvip/operators/lidu.py:4-8), which is
the out-variant op ``lidu_fused_batch_get_prepare_mtp_out``
(csrc/operators/lidu/torch_extension/csrc/lidu_fused_batch_get_prepare_mtp_ops.cpp:195-270):
20 tensors and four integers in the reference's order, the six outputs returned. The
tensor checks mirror the reference host op (:41-190) and raise ValueError. The work is
enqueued on torch's current stream of the tensors' device through ``kvip_hip_lidu``
(libkvip_hip.so).

Workspace: the kernels need per-request scratch (kvip_hip_lidu_workspace_bytes). It comes
from the caller (``workspace=``), from the device's reserved buffer (``lidu_reserve(device,
max_batch)`` at bind time: one buffer serves every batch up to max_batch), or, for an
eager call with neither, from a buffer the module grows on first use. A call under hipGraph
capture never allocates: without a caller or reserved workspace large enough it raises.

`lidu_prepare` is the allocating variant ``lidu_fused_batch_get_prepare_mtp`` (:272-300).

`register_torch_ops()` (run when this module is imported) defines the reference's two
operators in the ``nanovllm_dsa`` namespace with the reference's schemas (:374-399), for
callers that look them up as ``torch.ops.nanovllm_dsa.*`` (the reference's harness,
tests/operators/lifetch/support/execution.py:678-683): the CUDA (HIP) kernels are this
module's `lidu` / `lidu_prepare`, and the Meta kernels give the output shapes for tracing
(as the reference's Meta implementation does, :320-372).
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

_WORKSPACES = {}  # device -> int32 workspace tensor (reserved or grown eagerly)


def _torch():
    import torch

    return torch


def workspace_bytes(batch):
    """Bytes of LIDU workspace a batch of `batch` requests needs."""
    return int(abi.load_library().kvip_hip_lidu_workspace_bytes(int(batch)))


def lidu_reserve(device, max_batch):
    """Allocate (once) the device's LIDU workspace for batches of up to `max_batch`
    requests, so that later calls, captured ones included, allocate nothing. Returns it."""
    torch = _torch()
    device = abi.device_of(torch, device)
    nbytes = workspace_bytes(max_batch)
    ws = _WORKSPACES.get(str(device))
    if ws is None or ws.numel() * 4 < nbytes:
        ws = torch.empty((nbytes + 3) // 4, dtype=torch.int32, device=device)
        _WORKSPACES[str(device)] = ws
    return ws


def _workspace(torch, device, batch, workspace):
    need = workspace_bytes(batch)
    if workspace is not None:
        if (workspace.dtype != torch.int32 or workspace.device != device or not workspace.is_contiguous()
                or workspace.numel() * 4 < need):
            raise ValueError(f"lidu: workspace must be a contiguous int32 tensor of at least {need} bytes on {device}")
        return workspace
    ws = _WORKSPACES.get(str(device))
    if ws is not None and ws.numel() * 4 >= need:
        return ws
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"lidu: no workspace of {need} bytes is reserved for this batch on {device}; call "
                           f"kvip_amd.lidu_reserve(device, max_batch) before capture or pass workspace=")
    return lidu_reserve(device, batch)


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
         resident_seq_lengths, profiling, layer_id, num_layers, max_num_reqs, qcap, *, workspace=None):
    """Run the LIDU transaction; token_to_slot_pool, slot_to_token_pool, eviction_cursors and the
    outputs are written in place. Returns (destination_slots, miss_counts, indices, offsets,
    output_indices, resident_seq_lengths). workspace: an optional caller-owned int32 tensor of
    at least workspace_bytes(B) bytes."""
    torch = _torch()
    batch, packed = _check_inputs(
        torch, topk_indices, actual_seq_lengths_query, req_pool_entries, token_to_slot_pool, slot_to_token_pool,
        eviction_cursors, cache_tokens, candidate_lens, miss_slots, miss_slot_bitmap, resident_block_table,
        logical_seq_lengths, profile_enabled, layer_id, num_layers, max_num_reqs, qcap)
    _check_outputs(torch, topk_indices, batch, destination_slots, miss_counts, indices, offsets, output_indices,
                   resident_seq_lengths, profiling)
    lib = abi.load_library()
    device = abi.device_of(torch, topk_indices.device)
    ws = _workspace(torch, device, batch, workspace)
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


# The reference operators' schemas (lidu_fused_batch_get_prepare_mtp_ops.cpp:374-399).
_SCHEMA = (
    "lidu_fused_batch_get_prepare_mtp(Tensor topk_indices, Tensor actual_seq_lengths_query, "
    "Tensor req_pool_entries, Tensor(a!) token_to_slot_pool, Tensor(b!) slot_to_token_pool, "
    "Tensor(c!) eviction_cursors, Tensor cache_tokens, Tensor candidate_lens, Tensor miss_slots, "
    "Tensor miss_slot_bitmap, Tensor resident_block_table, Tensor logical_seq_lengths, Tensor profile_enabled, "
    "int layer_id, int num_layers, int max_num_reqs, int qcap) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
_SCHEMA_OUT = (
    "lidu_fused_batch_get_prepare_mtp_out(Tensor topk_indices, Tensor actual_seq_lengths_query, "
    "Tensor req_pool_entries, Tensor(a!) token_to_slot_pool, Tensor(b!) slot_to_token_pool, "
    "Tensor(c!) eviction_cursors, Tensor cache_tokens, Tensor candidate_lens, Tensor miss_slots, "
    "Tensor miss_slot_bitmap, Tensor resident_block_table, Tensor logical_seq_lengths, Tensor profile_enabled, "
    "Tensor(d!) destination_slots, Tensor(e!) miss_counts, Tensor(f!) indices, Tensor(g!) offsets, "
    "Tensor(h!) output_indices, Tensor(i!) resident_seq_lengths, Tensor(j!) profiling, int layer_id, "
    "int num_layers, int max_num_reqs, int qcap) -> (Tensor(d!), Tensor(e!), Tensor(f!), Tensor(g!), "
    "Tensor(h!), Tensor(i!))")
_TORCH_LIBRARY = None


def _prepare_meta(topk_indices, actual_seq_lengths_query, *rest):
    torch = _torch()
    batch = actual_seq_lengths_query.shape[0]
    cap = batch * MISS_CAPACITY
    dev = topk_indices.device
    return (torch.empty(topk_indices.shape, dtype=torch.int32, device=dev),
            torch.empty(batch + 1, dtype=torch.int32, device=dev), torch.empty(cap, dtype=torch.int32, device=dev),
            torch.empty(cap, dtype=torch.int32, device=dev), torch.empty(cap, dtype=torch.int32, device=dev),
            torch.empty(batch, dtype=torch.int32, device=dev))


def _out_meta(*args):
    return tuple(args[13:19])


def register_torch_ops():
    """Define nanovllm_dsa::lidu_fused_batch_get_prepare_mtp and _out with the reference's
    schemas, with CUDA (HIP) and Meta kernels. Idempotent."""
    global _TORCH_LIBRARY
    if _TORCH_LIBRARY is not None:
        return _TORCH_LIBRARY
    torch = _torch()
    lib = torch.library.Library("nanovllm_dsa", "FRAGMENT")
    lib.define(_SCHEMA)
    lib.define(_SCHEMA_OUT)
    lib.impl("lidu_fused_batch_get_prepare_mtp", lidu_prepare, "CUDA")
    lib.impl("lidu_fused_batch_get_prepare_mtp_out", lidu, "CUDA")
    lib.impl("lidu_fused_batch_get_prepare_mtp", _prepare_meta, "Meta")
    lib.impl("lidu_fused_batch_get_prepare_mtp_out", _out_meta, "Meta")
    _TORCH_LIBRARY = lib
    return lib


register_torch_ops()
