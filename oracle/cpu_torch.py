"""Multi-threaded torch-CPU restatement of one decode query row of the hot path: decode the
fp8 operands to float32, LI keys, TopK-2048, Fetch gather.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): bench.py's cpu_baseline leg times it
on the host as the CPU baseline, and tests/test_oracle_cpu_torch.py pins it against
oracle/indexer.py. It is never imported by kvip_amd.

Same algorithm as oracle/indexer.py, arranged for a multi-core host: the per-head dot
products and the weighted head reduction run as two BLAS products (float32, threaded by
torch), where oracle.indexer.li_scores forms each dot product exactly in float64 and
reduces heads in the device's even/odd FMA order. Keys therefore agree with the oracle
except where a score's last float32 bits decide a bf16 rounding; the tests bound that
share. Reference formulas: indexer_score.h:60-140 and :384-426 (ReLU, w * qscale, head
sum, key scale), workloads.py:233-235 (bf16 half away from zero), score_common.h:66-97
(sortable key), topk.h:155-187 with topk_common.h:1000-1067 (one GT-then-EQ pass),
kvaf-ubmem-device-get.patch:41-90 (row gather).
"""
from __future__ import annotations

TOPK = 2048
BLOCK_TOKENS = 128


def sortable_keys(torch, scores):
    """float32 scores -> int32 holding the uint16 sortable key of the bf16 rounding (ties
    away from zero)."""
    bits = scores.contiguous().view(torch.int32).to(torch.int64)
    bf = ((bits + 0x8000) >> 16) & 0xFFFF
    bf = torch.where(bf == 0x7FC0, torch.full_like(bf, 0xFFFF), bf)
    key = torch.where((bf & 0x8000) != 0, (~bf) & 0xFFFF, bf ^ 0x8000)
    return key.to(torch.int32)


def li_keys(torch, query, keys, weights, query_scale=None, key_scale=None):
    """query [heads, 128], keys [tokens, 128] float32; weights, query_scale [heads];
    key_scale [tokens] -> int32 sortable keys [tokens]."""
    w = weights.float()
    if query_scale is not None:
        w = w * query_scale.float()
    qk = torch.mm(query, keys.t())            # [heads, tokens]
    score = torch.mv(qk.clamp_min_(0).t(), w)  # sum_h ReLU(qk_h) * w'_h
    if key_scale is not None:
        score = score * key_scale
    return sortable_keys(torch, score)


def topk(torch, keys, valid, topk=TOPK):
    """Single-pass reference order: positions with key > kth ascending, then positions
    with key == kth ascending, first topk; rows shorter than topk list 0..valid-1."""
    out = torch.full((topk,), -1, dtype=torch.int64)
    if valid <= 0:
        return out
    if valid < topk:
        out[:valid] = torch.arange(valid)
        return out
    row = keys[:valid]
    kth = torch.kthvalue(row, valid - topk + 1).values
    gt = torch.nonzero(row > kth).flatten()
    eq = torch.nonzero(row == kth).flatten()
    return torch.cat((gt, eq))[:topk]


def fetch_rows(torch, kv_rows, pages, selected):
    """kv_rows [blocks * 128, row_bytes] uint8; pages: the request's block-table row;
    selected: token positions (-1 = no row) -> [len(selected), row_bytes], zeros for -1."""
    live = selected >= 0
    pos = selected.clamp_min(0)
    rows = pages[pos // BLOCK_TOKENS].to(torch.int64) * BLOCK_TOKENS + pos % BLOCK_TOKENS
    out = kv_rows.index_select(0, rows)
    out[~live] = 0
    return out


def decode_row(torch, q_raw, k_raw, weights, query_scale, key_scale, kv_rows, pages, valid):
    """One decode query row end to end from fp8 bytes: q_raw [heads, 128] and k_raw
    [valid, 128] uint8 (e4m3fn codes), key_scale [valid] or None -> (selected, rows)."""
    q = q_raw.view(torch.float8_e4m3fn).float()
    k = k_raw.view(torch.float8_e4m3fn).float()
    keys = li_keys(torch, q, k, weights, query_scale, key_scale)
    sel = topk(torch, keys, valid)
    return sel, fetch_rows(torch, kv_rows, pages, sel)
