"""`kvip_amd.update_abc`: ABC ring maps on the device (python/kvip/cache/abc.py:5-33).

Same signature and in-place semantics as the reference: for every group and each of its
first `requests` descriptor rows (layer, owner, begin, end), token_to_slot[layer, owner,
begin:end] = history + t % tail and the ring slot_to_token[layer, owner,
history:history+tail] holds the range's tokens (later tokens win, -1 elsewhere). The
reference's CPU branch is its golden; here the tensors must be on the GPU (there is no
CPU path: the oracle of tests/ holds the CPU restatement).
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi


def update_abc(token_to_slot, slot_to_token, descriptors, requests, history, tail, *, status=None):
    torch = _torch()
    for name, t in (("token_to_slot", token_to_slot), ("slot_to_token", slot_to_token),
                    ("descriptors", descriptors)):
        if t.device.type != "cuda":
            raise ValueError(f"update_abc: {name} must be a GPU tensor (kvip_amd has no CPU path)")
        if t.dtype != torch.int32 or not t.is_contiguous() or t.dim() != 3:
            raise ValueError(f"update_abc: {name} must be a contiguous int32 3-D tensor")
    if token_to_slot.shape[:2] != slot_to_token.shape[:2] or descriptors.shape[2] != 4:
        raise ValueError("update_abc: maps must share [layers, pool] and descriptors be [groups, rows, 4]")
    if not 0 <= requests <= descriptors.shape[1] or tail < 1 or history < 0 or history + tail > slot_to_token.shape[2]:
        raise ValueError("update_abc: requests/history/tail outside the tensors")
    lib = abi.load_library()
    args = abi.AbcArgs(
        token_to_slot=abi.ptr(token_to_slot), slot_to_token=abi.ptr(slot_to_token),
        descriptors=abi.ptr(descriptors), status=abi.ptr(status), groups=descriptors.shape[0],
        rows=descriptors.shape[1], requests=requests, layers=token_to_slot.shape[0], pool=token_to_slot.shape[1],
        t2s_tokens=token_to_slot.shape[2], s2t_tokens=slot_to_token.shape[2], history=history, tail=tail,
    )
    abi.check(lib.kvip_hip_update_abc(ctypes.byref(args), abi.stream_handle(torch, token_to_slot.device)),
              "update_abc")


def _torch():
    import torch

    return torch
