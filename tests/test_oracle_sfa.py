"""The sparse-attention oracle (oracle/sfa.py) pinned on the CPU: row unpacking against
torch's own fp8 e4m3 and bf16 decoders, payload known answers, and attention closed forms;
plus the host-side checks of kvip_amd.SparseAttention."""
import numpy as np
import pytest

from oracle import sfa


def test_payload_known_answers():
    rows = sfa.kv_payload(0, [0, 1])
    # Token 0, layer 0: nope byte c is code[c % 7], rope c is 0x3E80 | c, scales 1/32..1/4.
    assert rows.shape == (2, 656)
    assert rows[0, :9].tolist() == [0xC4, 0xC0, 0xB8, 0, 0x38, 0x40, 0x44, 0xC4, 0xC0]
    assert rows[0, 512:640].view("<u2")[:3].tolist() == [0x3E80, 0x3E81, 0x3E82]
    assert rows[0, 640:].view("<f4").tolist() == [0.03125, 0.0625, 0.125, 0.25]
    # Token 1 shifts the first 8 nope bytes (shift 0) by one code and keeps byte 8's group
    # (shift 1: 1 >> 1 = 0).
    assert rows[1, :2].tolist() == [0xC0, 0xB8] and rows[1, 8] == rows[0, 8]
    assert sfa.kv_payload(1, [0])[0, 0] == 0  # layer 1 adds 3 to the code index


def test_unpack_matches_torch_decoders():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    rows = sfa.kv_payload(2, rng.integers(0, 1 << 17, 40))
    key, value = sfa.unpack_rows(rows)
    nope = torch.from_numpy(rows[:, :512].copy()).view(torch.float8_e4m3fn).float().numpy()
    scales = rows[:, 640:].copy().view("<f4")
    want_nope = nope * np.repeat(scales, 128, axis=1)
    rope = torch.from_numpy(rows[:, 512:640].copy().view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(value, want_nope)
    assert np.array_equal(key, np.concatenate((want_nope, rope), axis=1))


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(4).standard_normal(100000).astype(np.float32)
    assert np.array_equal(sfa._bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    rows = sfa.kv_payload(0, rng.permutation(4096)[:2048])
    _, value = sfa.unpack_rows(rows)
    # Zero queries: uniform probabilities 1/2048 (exact in bf16) -> the mean value.
    out = sfa.sparse_attention(np.zeros((4, 576), np.float32), rows, 576 ** -0.5)
    assert np.allclose(out, value.mean(axis=0), rtol=1e-5, atol=1e-7)
    # One dominant token: its probability rounds to 1, every other to 0.
    key, _ = sfa.unpack_rows(rows)
    q = np.zeros((1, 576), np.float32)
    q[0] = key[17] * 1000.0
    logits = np.sort(key @ q[0])
    assert logits[-1] - logits[-2] > 200.0  # exp(-200) is 0 in float32
    out = sfa.sparse_attention(q, rows, 1.0)
    assert np.array_equal(out[0], value[int(np.argmax(key @ q[0]))])
    # Order of the rows does not matter (up to float32 summation order).
    q = rng.uniform(-0.2, 0.2, (8, 576)).astype(np.float32)
    perm = rng.permutation(2048)
    assert np.allclose(sfa.sparse_attention(q, rows, 0.05), sfa.sparse_attention(q, rows[perm], 0.05), rtol=1e-5,
                       atol=1e-5)
    # Against the softmax identity in float64 (bf16 probabilities: relative error <= 2^-8).
    logits = q.astype(np.float64) @ key.T.astype(np.float64) * 0.05
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    want = (p / p.sum(axis=1, keepdims=True)) @ value.astype(np.float64)
    assert np.allclose(sfa.sparse_attention(q, rows, 0.05), want, rtol=1e-2, atol=2e-3)


def test_sparse_attention_host_checks():
    torch = pytest.importorskip("torch")
    from kvip_amd.operators.sfa import SparseAttention

    with pytest.raises(ValueError):
        SparseAttention(torch, rows=3, heads=8, device="cpu", rows_per_request=2)
    with pytest.raises(ValueError):
        SparseAttention(torch, rows=4, heads=129, device="cpu")
