"""The torch-CPU restatement timed as bench.py's CPU baseline (oracle/cpu_torch.py) against
the numpy oracle: bf16 rounding and sortable keys bit-exact, TopK order exact, gather
byte-exact, LI keys identical except for last-bit rounding differences of the float32
reduction order."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import cpu_torch
from oracle import indexer as ref


def test_sortable_keys_match_the_oracle():
    rng = np.random.default_rng(5)
    vals = rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 20, 20000)
    # ties of the bf16 rounding (low half exactly 0x8000), signed zeros, tiny and huge values
    ties = (rng.integers(0, 1 << 15, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    special = np.array([0.0, -0.0, 1e-40, -1e-40, 3.0e38, -3.0e38, 1.0, -1.0], np.float32)
    vals = np.concatenate([vals.astype(np.float32), ties, special])
    got = cpu_torch.sortable_keys(torch, torch.from_numpy(vals)).numpy()
    want = ref.sortable_key(ref.bf16_round_half_away(vals)).astype(np.int64)
    assert np.array_equal(got, want)


def test_li_keys_agree_with_the_oracle():
    rng = np.random.default_rng(6)
    heads, tokens = 64, 3000
    q_raw = (rng.integers(0, 256, (heads, 128)) & 0x77).astype(np.uint8)
    k_raw = (rng.integers(0, 256, (tokens, 128)) & 0x77).astype(np.uint8)
    w = (rng.standard_normal(heads) / 8).astype(np.float32)
    qs = (rng.random(heads) + 0.5).astype(np.float32)
    ks = (rng.random(tokens) * 1.5 + 0.5).astype(np.float32)
    want = ref.li_keys(ref.fp8_e4m3_decode(q_raw), ref.fp8_e4m3_decode(k_raw), w, qs, ks)
    q = torch.from_numpy(q_raw).view(torch.float8_e4m3fn).float()
    k = torch.from_numpy(k_raw).view(torch.float8_e4m3fn).float()
    got = cpu_torch.li_keys(torch, q, k, torch.from_numpy(w), torch.from_numpy(qs), torch.from_numpy(ks)).numpy()
    assert ref.identical_share(got[None].astype(np.uint16), want[None], [tokens]) >= 0.99
    # every key within one bf16 step of the oracle's
    assert np.abs(got.astype(np.int64) - want.astype(np.int64)).max() <= 1


@pytest.mark.parametrize("valid", [0, 1, 2047, 2048, 5000])
def test_topk_order_matches_the_oracle(valid):
    rng = np.random.default_rng(valid + 7)
    keys = rng.integers(0x8000, 0x8000 + 40, size=max(valid, 1)).astype(np.uint16)  # heavy ties
    got = cpu_torch.topk(torch, torch.from_numpy(keys.astype(np.int32)), valid).numpy()
    assert np.array_equal(got, ref.topk_reference(keys, valid))


def test_fetch_rows_match_the_oracle():
    rng = np.random.default_rng(8)
    kv = rng.integers(0, 256, (6, 128, 656)).astype(np.uint8)
    table = np.array([[4, 1, 5, 0]], np.int32)
    sel = rng.choice(4 * 128, 2048, replace=True).astype(np.int64)
    sel[::97] = -1
    want = ref.fetch_gather(kv, table, sel[None])[0]
    got = cpu_torch.fetch_rows(torch, torch.from_numpy(kv.reshape(-1, 656)), torch.from_numpy(table[0]),
                               torch.from_numpy(sel)).numpy()
    assert np.array_equal(got, want)
