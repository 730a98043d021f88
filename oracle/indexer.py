"""CPU restatement of the lightning-indexer score, TopK-2048 and Fetch gather.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by kvip_amd.

Reference paths are relative to the KVIP reference tree.
"""
from __future__ import annotations

import numpy as np

TOPK = 2048
BLOCK_TOKENS = 128
INDEX_DIM = 128
TOKEN_BYTES = 656
TRUNK_SINGLE_ROW = 16384  # trunkLen_ when s1BaseSize == 2 or topk-only
TRUNK_Q4 = 8192           # trunkLen_ otherwise (op_kernel/indexer/indexer_vector.h:375-379)


# ----------------------------------------------------------------------------
# Element decoding
# ----------------------------------------------------------------------------
def fp8_e4m3_decode(raw):
    """OCP fp8 e4m3fn bytes -> float32.

    Follows tests/operators/lifetch/support/workloads.py:505-515 (`unpack`: sign bit 7,
    exponent bits 3..6 with bias 7, mantissa bits 0..2, subnormal = m/8 * 2^-6), plus the
    e4m3fn NaN codes 0x7F/0xFF. Pinned by tests/test_oracle_indexer.py against torch's
    independent float8_e4m3fn conversion on all 256 codes.
    """
    raw = np.asarray(raw, dtype=np.uint8)
    sign = np.where(raw & 0x80, -1.0, 1.0)
    exponent = ((raw >> 3) & 15).astype(np.int32)
    mantissa = (raw & 7).astype(np.float64)
    value = np.where(exponent == 0, mantissa / 8.0 * 2.0 ** -6, (1.0 + mantissa / 8.0) * np.exp2(exponent - 7.0))
    value = sign * value
    value = np.where((raw & 0x7F) == 0x7F, np.nan, value)
    return value.astype(np.float32)


def bf16_decode(bits):
    """bf16 bit patterns -> float32 (upper half of the float32 word)."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def bf16_round_half_away(values):
    """float32 -> bf16 bits with Ascend CAST_ROUND (ties away from zero).

    workloads.py:233-235 and :1235: ``(score.view(uint32) + 0x8000) >> 16``. Pinned by
    tests against torch's round-to-nearest-even on every non-tie input and by known
    tie answers (a tie always moves away from zero).
    """
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    return ((bits.astype(np.uint64) + 0x8000) >> 16).astype(np.uint16)


def sortable_key(bf16_bits):
    """bf16 bits -> order-preserving uint16 key.

    op_kernel/indexer/score_common.h:66-97 (FloatToSortableKey: canonical NaN 0x7FC0 ->
    0xFFFF, then negative -> ~bits, non-negative -> bits ^ 0x8000); same as
    workloads.py:1237 for non-NaN input. Pinned by the known answers of
    support/correctness.py:198-202 (0x8000 = +0, 0xC200 = +32) and by a brute-force
    order check over all non-NaN bf16 values.
    """
    bits = np.asarray(bf16_bits, dtype=np.uint16)
    bits = np.where(bits == 0x7FC0, np.uint16(0xFFFF), bits)
    return np.where(bits & 0x8000, ~bits, bits ^ np.uint16(0x8000)).astype(np.uint16)


def score_values(keys):
    """Sortable keys -> float32 score values (workloads.py:526-531)."""
    keys = np.asarray(keys, dtype=np.uint16)
    bits = np.where(keys & 0x8000, keys ^ 0x8000, ~keys).astype(np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------
# LI score
# ----------------------------------------------------------------------------
def identical_share(got_keys, want_keys, valid, floor=3e-2):
    """Share of bit-identical keys among the valid keys whose oracle |score| is at least
    `floor` of the row's largest |score|. A checker's statistic, not part of the
    algorithm: the device's fp8 dot products are not correctly rounded fp32, so scores that
    cancel to near zero (where a bf16 ulp is far below that absolute error) may differ in
    their last bits; every key is held to the score tolerance separately."""
    same = total = 0
    for r, v in enumerate(valid):
        if v == 0:
            continue
        w = np.abs(score_values(want_keys[r, :v]).astype(np.float64))
        keep = w >= floor * w.max()
        same += int(np.sum(got_keys[r, :v][keep] == want_keys[r, :v][keep]))
        total += int(keep.sum())
    return same / max(total, 1)


def _fma32(a, b, c):
    """float32 a*b + c rounded once; emulated in float64 (a*b is exact there, the add
    can double-round in rare last-bit cases)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def li_scores(query, keys, weights, query_scale=None, key_scale=None):
    """Lightning-indexer scores of one query row against a run of tokens.

    query [heads, 128] and keys [tokens, 128] are float32 values already decoded from
    fp8/bf16; weights [heads] (bf16 or fp32 values); query_scale [heads]; key_scale
    [tokens]. Device order of op_kernel/indexer/indexer_score.h:384-426 with the loop
    of :60-103 and the finalize of :105-140:
      qk_h    = fp32 dot product (the cube MMAD, indexer_cube.h:161-322)
      w'_h    = w_h * qscale_h                          (fp32 multiply)
      acc_e   = FMA chain of ReLU(qk_h) * w'_h over even heads, ascending
      acc_o   = the same over odd heads
      score   = (acc_e + acc_o) * kscale_t
    The fp32 dot product is formed exactly in float64 and rounded once (exact for fp8
    inputs). Pinned by the exact-binary fixture of workloads.py:196-283 and by
    closed-form ReLU/sign cases in tests/test_oracle_indexer.py.
    """
    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    heads = q.shape[0]
    qk = (q @ k.T).astype(np.float32)  # [heads, tokens]
    w = np.asarray(weights, dtype=np.float32).reshape(heads)
    qs = np.ones(heads, np.float32) if query_scale is None else np.asarray(query_scale, np.float32).reshape(heads)
    wq = (w * qs).astype(np.float32)
    acc = [np.zeros(k.shape[0], np.float32), np.zeros(k.shape[0], np.float32)]
    for h in range(heads):
        acc[h & 1] = _fma32(np.maximum(qk[h], np.float32(0)), np.float32(wq[h]), acc[h & 1])
    score = (acc[0] + acc[1]).astype(np.float32)
    if key_scale is not None:
        score = (score * np.asarray(key_scale, np.float32)).astype(np.float32)
    return score


def li_keys(query, keys, weights, query_scale=None, key_scale=None):
    """Sortable uint16 keys of li_scores (indexer_score.h:105-140 + score_common.h:66-97)."""
    return sortable_key(bf16_round_half_away(li_scores(query, keys, weights, query_scale, key_scale)))


def paged_rows(cache, block_table_row, tokens):
    """Rows of `tokens` from a paged cache [blocks, 128, ...] through one block-table row."""
    tokens = np.asarray(tokens, dtype=np.int64)
    return cache[np.asarray(block_table_row)[tokens // BLOCK_TOKENS], tokens % BLOCK_TOKENS]


def decode_keys_paged(query, weights, query_scale, keys, key_scale, block_table, seq_lens,
                      rows_per_request=1, query_ends=None, key_stride=None):
    """Score every valid token of every query row of a paged decode batch.

    query [rows, heads, 128] float32 values; keys [blocks, 128, 128] float32 values;
    key_scale [blocks, 128] or None; block_table [batch, max_blocks]; valid(r) =
    min(seq_lens[b], query_ends[r]). Returns (keys [rows, key_stride] uint16 with zeros
    past valid, valid [rows]).
    """
    rows = query.shape[0]
    batch, max_blocks = block_table.shape
    stride = key_stride or max_blocks * BLOCK_TOKENS
    out = np.zeros((rows, stride), np.uint16)
    valid = np.zeros(rows, np.int64)
    for r in range(rows):
        b = r // rows_per_request
        v = int(seq_lens[b]) if query_ends is None else min(int(seq_lens[b]), int(query_ends[r]))
        v = max(0, min(v, max_blocks * BLOCK_TOKENS))
        valid[r] = v
        if v == 0:
            continue
        tokens = np.arange(v)
        k = paged_rows(keys, block_table[b], tokens)
        ks = None if key_scale is None else paged_rows(key_scale, block_table[b], tokens)
        qs = None if query_scale is None else query_scale[r]
        out[r, :v] = li_keys(query[r], k, weights[r], qs, ks)
    return out, valid


def prefill_visible(cu_seqlens_q, seq_lens_k):
    """Visible key positions of every packed query row under the right-down causal mask
    (sparse_mode 3 of the native indexer the reference's selector calls for prefill rows,
    python/kvip/adapters/vllm/selector.py:126-154): local row j of a sequence with q_len
    rows and k_len keys sees positions t < clamp(k_len - q_len + j + 1, 0, k_len)."""
    out = []
    for s in range(len(seq_lens_k)):
        q_len = int(cu_seqlens_q[s + 1] - cu_seqlens_q[s])
        k_len = int(seq_lens_k[s])
        for j in range(q_len):
            out.append(max(0, min(k_len - q_len + j + 1, k_len)))
    return np.array(out, np.int64)


def prefill_keys_paged(query, weights, query_scale, keys, key_scale, block_table, cu_seqlens_q, seq_lens_k,
                       key_stride):
    """Keys of packed prefill rows: row r of sequence s scores positions [0, vis(r)) of
    that sequence's paged keys with the decode formula (li_keys). Returns (keys
    [rows, key_stride] uint16 with zeros past vis, vis [rows])."""
    vis = prefill_visible(cu_seqlens_q, seq_lens_k)
    out = np.zeros((len(vis), key_stride), np.uint16)
    for s in range(len(seq_lens_k)):
        k_len = int(seq_lens_k[s])
        tokens = np.arange(k_len)
        k = paged_rows(keys, block_table[s], tokens)
        ks = None if key_scale is None else paged_rows(key_scale, block_table[s], tokens)
        for r in range(int(cu_seqlens_q[s]), int(cu_seqlens_q[s + 1])):
            v = int(vis[r])
            if v == 0:
                continue
            qs = None if query_scale is None else query_scale[r]
            out[r, :v] = li_keys(query[r], k[:v], weights[r], qs, None if ks is None else ks[:v])
    return out, vis


# ----------------------------------------------------------------------------
# TopK-2048
# ----------------------------------------------------------------------------
def _select_gt_eq(values, topk):
    """One LiTopKVF pass (op_kernel/indexer/topk_common.h:1137-1187): positions of the
    values > kth in position order (FindIdxGTOutputVFImpl, :1000-1032) followed by the
    positions == kth in position order (FindIdxEQOutputVFImpl, :1037-1067), first topk."""
    kth = np.partition(values, len(values) - topk)[len(values) - topk]
    gt = np.flatnonzero(values > kth)
    eq = np.flatnonzero(values == kth)
    return np.concatenate((gt, eq))[:topk]


def topk_reference(keys, valid, topk=TOPK, trunk=None):
    """TopK-2048 of one row of sortable keys, reproducing the reference's output order.

    QLIVector::ProcessTopK (op_kernel/indexer/indexer_vector.h:799-973): valid <= 0 ->
    all -1; valid < topk -> [0..valid-1, -1...] (:943-957); otherwise LITopk<uint16_t>
    (topk.h:155-187): one GT-then-EQ pass when valid <= trunk, else trunk 0 is selected
    and each later trunk is merged as [prior winners' keys, trunk keys] and re-selected,
    positions < topk mapping to prior winners (FindRealIndexVFImpl,
    topk_common.h:1094-1122). Zero padding to 256-element alignment is never selected
    (key 0 is below every finite score). trunk=None means a single pass.
    """
    keys = np.asarray(keys, dtype=np.uint16)
    out = np.full(topk, -1, np.int64)
    if valid <= 0:
        return out
    if valid < topk:
        out[:valid] = np.arange(valid)
        return out
    row = keys[:valid].astype(np.int64)
    if trunk is None or valid <= trunk:
        return _select_gt_eq(row, topk)
    winners = _select_gt_eq(row[:trunk], topk)
    for start in range(trunk, valid, trunk):
        part = row[start:start + trunk]
        merged = np.concatenate((row[winners], part))
        pos = _select_gt_eq(merged, topk)
        winners = np.where(pos < topk, winners[np.minimum(pos, topk - 1)], pos - topk + start)
    return winners


def topk_set_rule(keys, valid, topk=TOPK):
    """Closed form of the selected set: the first topk tokens of the order
    (key desc, token asc). Used to pin topk_reference (any trunk size)."""
    if valid < topk:
        return topk_reference(keys, valid, topk)
    row = np.asarray(keys, dtype=np.int64)[:valid]
    order = np.lexsort((np.arange(valid), -row))
    return order[:topk]


def validate_topk_band(selected, scores, topk=TOPK):
    """support/correctness.py:22-36: a selection is accepted when it holds topk unique
    in-range tokens, none below cutoff - tol and every score above cutoff + tol, with
    tol one bf16 spacing of the cutoff (CPU/device reduction differences)."""
    selected = np.asarray(selected)
    row = np.asarray(scores, dtype=np.float32)
    if selected.min() < 0 or selected.max() >= len(row) or len(np.unique(selected)) != topk:
        return False
    cutoff = np.partition(row, -topk)[-topk]
    tol = max(float(abs(cutoff)) * 2 ** -7, float(np.finfo(np.float32).tiny))
    if row[selected].min() < cutoff - tol:
        return False
    mandatory = np.flatnonzero(row > cutoff + tol)
    return bool(np.isin(mandatory, selected).all())


# ----------------------------------------------------------------------------
# Fetch gather and KV payload
# ----------------------------------------------------------------------------
def fetch_gather(kv_cache, block_table, topk, rows_per_request=1):
    """Byte gather of the selected KV rows: out[r, i] = kv row topk[r, i] of request
    r // rows_per_request, zeros for -1 (descriptor semantics of
    patches/kvaf-ubmem-device-get.patch:41-90: dst = output + index * token_bytes,
    src = the token's row). kv_cache [blocks, 128, row_bytes] uint8."""
    rows = topk.shape[0]
    row_bytes = kv_cache.shape[-1]
    out = np.zeros((rows, topk.shape[1], row_bytes), np.uint8)
    for r in range(rows):
        ids = np.asarray(topk[r], np.int64)
        live = ids >= 0
        b = r // rows_per_request
        out[r, live] = paged_rows(kv_cache, block_table[b], ids[live])
    return out


def identity_rows(tokens, row_bytes=TOKEN_BYTES, salt=0):
    """Synthetic KV rows whose every byte is a function of (token, byte column, salt),
    so a row gathered from the wrong token, block or offset is detected byte-exactly.
    Plays the role of the reference's identity payload (workloads.py:493-502); the
    pattern itself is this build's own (a multiplicative hash of token and column)."""
    tokens = np.asarray(tokens, dtype=np.uint64).reshape(-1, 1)
    columns = np.arange(row_bytes, dtype=np.uint64)[None, :]
    mixed = (tokens * np.uint64(0x9E3779B1) + columns * np.uint64(0x85EBCA77) + np.uint64(salt) * np.uint64(0xC2B2AE3D))
    return ((mixed >> np.uint64(13)) & np.uint64(0xFF)).astype(np.uint8)
