"""CPU restatement of the sparse-attention consumer check. TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

kv_payload        - the deterministic 656-byte KV rows of the reference's workloads
                    (tests/operators/lifetch/support/workloads.py:493-502)
unpack_rows       - key [nope * scale, rope] and value nope * scale of rows (:505-515)
sparse_attention  - the logical-token oracle of check_sfa (correctness.py:278-291): fp32
                    logits, softmax, probabilities rounded to bf16, product with the values
Pinned in tests/test_oracle_sfa.py: unpack against torch's independent fp8 e4m3 and bf16
decoders, payload known answers, attention closed forms (uniform logits give the mean value,
a dominant token gives its value, order invariance, the softmax identity in float64).
"""
from __future__ import annotations

import numpy as np

from oracle.indexer import fp8_e4m3_decode

ROW = 656
_CODES = np.asarray([0xC4, 0xC0, 0xB8, 0, 0x38, 0x40, 0x44], np.uint8)
_SCALES = np.asarray([0.03125, 0.0625, 0.125, 0.25], "<f4")


def kv_payload(pool_layer, tokens):
    """uint8 [len(tokens), 656]: nope byte c of token t is a fixed code chosen by
    ((t >> ((c // 8) % 18)) + c + 3 * pool_layer) mod 7, rope value c is the bf16 pattern
    0x3E80 | ((t >> ((c // 4) % 18)) + c + 11 * pool_layer) & 127, scales 1/32 .. 1/4."""
    t = np.asarray(tokens, np.int64).reshape(-1, 1)
    c = np.arange(512, dtype=np.int64)[None, :]
    nope = _CODES[((t >> ((c // 8) % 18)) + c + pool_layer * 3) % 7]
    rc = np.arange(64, dtype=np.int64)[None, :]
    rope = (0x3E80 | (((t >> ((rc // 4) % 18)) + rc + pool_layer * 11) & 127)).astype("<u2").view(np.uint8)
    scales = np.broadcast_to(_SCALES, (len(t), 4)).copy().view(np.uint8)
    return np.concatenate((nope, rope, scales), axis=1)


def unpack_rows(rows):
    """rows uint8 [n, >= 656] -> (key float32 [n, 576], value float32 [n, 512])."""
    rows = np.asarray(rows, np.uint8).reshape(-1, rows.shape[-1])[:, :ROW]
    scales = rows[:, 640:656].copy().view("<f4")
    nope = (fp8_e4m3_decode(rows[:, :512]) * np.repeat(scales, 128, axis=1)).astype(np.float32)
    rope = (rows[:, 512:640].copy().view("<u2").astype(np.uint32) << 16).view(np.float32)
    return np.concatenate((nope, rope), axis=1), nope


def _bf16(x):
    """Round float32 to bf16 (nearest even), returned as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def sparse_attention(query, rows, scale):
    """query float32 [heads, 576] (bf16 values); rows uint8 [n, 656] (the selected rows,
    n >= 1). Returns float32 [heads, 512]."""
    key, value = unpack_rows(rows)
    logits = (np.asarray(query, np.float32) @ key.T) * np.float32(scale)
    logits -= logits.max(axis=1, keepdims=True)
    prob = np.exp(logits)
    prob /= prob.sum(axis=1, keepdims=True)
    return _bf16(prob) @ value
