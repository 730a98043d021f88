"""Pins of the CPU oracle (oracle/indexer.py) against the reference's known answers,
closed forms and brute force, so that the oracle itself can be trusted as the
checker of the HIP kernels. Paths in comments are relative to the KVIP reference."""
import numpy as np
import pytest

from oracle import indexer as ref


# ---------------------------------------------------------------- element decoding
def test_fp8_decode_matches_torch_on_all_codes():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    ours = ref.fp8_e4m3_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(ours)
    assert np.array_equal(ours[ok], theirs[ok])
    # A few hand values: 0x38 = 1.0, 0x40 = 2.0, 0x44 = 3.0 (workloads.py:207 key codes).
    assert list(ref.fp8_e4m3_decode(np.array([0x38, 0x40, 0x44, 0xB8, 0x01], np.uint8))) == \
        [1.0, 2.0, 3.0, -1.0, 2.0 ** -9]


def test_bf16_round_half_away_known_answers_and_torch_on_non_ties():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = rng.standard_normal(200000).astype(np.float32) * np.float32(1e3) ** rng.uniform(-3, 3, 200000).astype(np.float32)
    bits = x.view(np.uint32)
    non_tie = (bits & 0xFFFF) != 0x8000
    rne = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ours = ref.bf16_round_half_away(x)
    assert np.array_equal(ours[non_tie], rne[non_tie])
    # Exact ties move away from zero (CAST_ROUND), unlike round-to-nearest-even.
    ties = np.array([0x3F808000, 0xBF808000, 0x3F818000, 0x40008000], np.uint32).view(np.float32)
    assert list(ref.bf16_round_half_away(ties)) == [0x3F81, 0xBF81, 0x3F82, 0x4001]


def test_sortable_key_known_answers():
    # support/correctness.py:198-202: key 0x8000 is +0 and 0xC200 is bf16 +32.
    assert ref.sortable_key(ref.bf16_round_half_away(np.float32([0.0, 32.0]))).tolist() == [0x8000, 0xC200]
    assert ref.sortable_key(np.array([0x8000, 0x7FC0, 0xFF80, 0x7F80], np.uint16)).tolist() == \
        [0x7FFF, 0x0000, 0x007F, 0xFF80]
    assert ref.score_values(np.array([0xC200, 0x8000], np.uint16)).tolist() == [32.0, 0.0]


def test_sortable_key_orders_every_bf16_value():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    values = ref.bf16_decode(bits)
    finite = ~np.isnan(values)
    keys = ref.sortable_key(bits[finite]).astype(np.int64)
    v = values[finite].astype(np.float64)
    order = np.argsort(keys)
    assert np.all(np.diff(v[order]) >= 0)  # key order is value order (-0 just below +0)
    assert len(np.unique(keys)) == len(keys)
    assert np.array_equal(ref.score_values(ref.sortable_key(bits[finite])).view(np.uint32) >> 16, bits[finite])


# ---------------------------------------------------------------- LI score
def exact_binary_fixture(tokens, queries, seed):
    """The construction of workloads.py:196-283 (own code): index-K values in {0,1,2,3}
    (fp8 codes 0, 0x38, 0x40, 0x44), one-hot 1.0 queries per head at column
    (h + 16 q) % 128, exact-binary query scales {0.5,1,2} and weights {1,2,0.5}, key
    scales U(0.25, 2). Every partial sum is exact, so the expected key is fixed by the
    float32 formula of the fixture whatever the accumulation order."""
    rng = np.random.default_rng(seed)
    values = rng.integers(0, 4, (tokens, 128), dtype=np.uint8)
    key_codes = np.array([0, 0x38, 0x40, 0x44], np.uint8)[values]
    head = np.arange(64)[None, :]
    qi = np.arange(queries)[:, None]
    qscale = np.array([0.5, 1.0, 2.0], np.float32)[(head + qi) % 3]
    weights = np.array([1.0, 2.0, 0.5], np.float32)[(head * 2 + qi) % 3]
    scale = rng.uniform(0.25, 2, tokens).astype(np.float32)
    query_codes = np.zeros((queries, 64, 128), np.uint8)
    expected = []
    for q in range(queries):
        cols = (np.arange(64) + q * 16) % 128
        query_codes[q, np.arange(64), cols] = 0x38
        score = (values[:, cols].astype(np.float32) * (weights[q] * qscale[q])).sum(-1) * scale
        expected.append(((score.view(np.uint32) + 0x8000) >> 16).astype(np.uint16))
    return query_codes, key_codes, weights, qscale, scale, np.stack(expected)


@pytest.mark.parametrize("seed", [73121, 7])
def test_li_score_exact_binary_fixture(seed):
    q, k, w, qs, ks, expected_bf16 = exact_binary_fixture(1024, 4, seed)
    kf = ref.fp8_e4m3_decode(k)
    for r in range(4):
        keys = ref.li_keys(ref.fp8_e4m3_decode(q[r]), kf, w[r], qs[r], ks)
        assert np.array_equal(keys, ref.sortable_key(expected_bf16[r]))


def test_li_score_relu_and_signed_weights_closed_form():
    # Head h sees dot = d_h; negative dots are dropped by ReLU, weights may be negative.
    heads = 64
    q = np.zeros((heads, 128), np.float32)
    q[np.arange(heads), np.arange(heads)] = 1.0
    k = np.zeros((3, 128), np.float32)
    k[0, :heads] = np.where(np.arange(heads) % 2, 3.0, -2.0)       # odd heads +3, even heads -2
    k[1, :heads] = -1.0                                             # all negative -> score +0
    k[2, 5] = 4.0                                                   # only head 5
    w = np.where(np.arange(heads) % 4 == 1, -0.5, 0.25).astype(np.float32)
    s = ref.li_scores(q, k, w, None, np.float32([1.0, 1.0, 2.0]))
    odd = np.arange(1, heads, 2)
    assert s[0] == np.float32(3.0 * w[odd].sum())
    assert s[1] == 0.0 and not np.signbit(s[1])
    assert s[2] == np.float32(4.0 * w[5] * 2.0)


# ---------------------------------------------------------------- TopK
def test_topk_edge_rules():
    keys = np.arange(5000, dtype=np.uint16)
    assert (ref.topk_reference(keys, 0) == -1).all()
    assert (ref.topk_reference(keys, -3) == -1).all()
    out = ref.topk_reference(keys, 100)
    assert out[:100].tolist() == list(range(100)) and (out[100:] == -1).all()
    # valid == 2048 goes through the select (GT-then-EQ order), not the identity path.
    rev = np.arange(2048, 0, -1).astype(np.uint16)
    rev[10] = rev[11]
    out = ref.topk_reference(rev, 2048)
    assert sorted(out.tolist()) == list(range(2048))


def test_topk_gt_then_eq_order_known_answer():
    keys = np.array([5, 9, 7, 9, 7, 7, 1, 9, 7], np.uint16)
    # top 5: 9,9,9 (GT 7) at 1,3,7 then the first two 7s at 2,4.
    assert ref.topk_reference(keys, len(keys), topk=5).tolist() == [1, 3, 7, 2, 4]


@pytest.mark.parametrize("valid,levels,trunk", [
    (20000, 65536, ref.TRUNK_SINGLE_ROW), (20000, 40, ref.TRUNK_SINGLE_ROW), (40000, 3, ref.TRUNK_Q4),
    (9000, 7, None), (131072, 300, ref.TRUNK_SINGLE_ROW)])
def test_topk_set_matches_closed_form_any_trunk(valid, levels, trunk):
    rng = np.random.default_rng(valid + levels)
    keys = (0x8000 + rng.integers(0, levels, valid)).astype(np.uint16)
    got = ref.topk_reference(keys, valid, trunk=trunk)
    want = ref.topk_set_rule(keys, valid)
    assert len(np.unique(got)) == 2048
    assert np.array_equal(np.sort(got), np.sort(want))


def _literal_trunk_topk(keys, valid, topk, trunk, align=256):
    """The reference's trunked TopK restated on explicit buffers, independently of the
    oracle's selection: QLIVector::ProcessTopK's trunk loop (indexer_vector.h:864-936: the
    first trunk alone, then [prior winners' keys, zero fill to the 256-aligned TopK count,
    the trunk's keys, zero fill to a multiple of 256]), LITopk<uint16_t>::operator()
    (topk.h:155-187), LiTopKVF (topk_common.h:1137-1187: the kth value is the
    (len - topk + 1)-th smallest of the buffer, then the positions above it and the
    positions equal to it, both in buffer order, first topk) and FindRealIndexVFImpl
    (:1094-1122: buffer index i > topk - 1 is position i + trunk start - aligned TopK
    count, else prior winner i)."""
    keys = [int(k) for k in keys]
    if valid <= 0:
        return [-1] * topk
    if valid < topk:
        return list(range(valid)) + [-1] * (topk - valid)
    up = lambda n: -(-n // align) * align
    topk_al = up(topk)

    def litopkvf(buf):
        kth = sorted(buf)[len(buf) - topk]
        idx = [i for i, v in enumerate(buf) if v > kth] + [i for i, v in enumerate(buf) if v == kth]
        idx = idx[:topk]
        return idx, [buf[i] for i in idx]

    loops = -(-valid // trunk)
    if loops == 1:
        buf = keys[:valid] + [0] * (up(valid) - valid)
        return litopkvf(buf)[0]
    his_idx, his_val = litopkvf(keys[:trunk])
    for loop in range(1, loops):
        vtl = valid % trunk if loop * trunk + trunk > valid else trunk
        buf = his_val + [0] * (topk_al - topk) + keys[loop * trunk:loop * trunk + vtl]
        buf += [0] * (up(len(buf)) - len(buf))
        idx, his_val = litopkvf(buf)
        base = loop * trunk - topk_al
        his_idx = [i + base if i > topk - 1 else his_idx[i] for i in idx]
    return his_idx


@pytest.mark.parametrize("seed", range(6))
def test_trunked_topk_order_equals_single_pass(seed):
    """The emission order of the reference's trunk merge (prior winners first) equals the
    single-pass GT-then-EQ order. Why: the kth key of a merge is the topk-th largest of
    the whole prefix scored so far, so it never decreases from one trunk to the next; a
    prior winner equal to an earlier kth can therefore never rise above a later kth, and
    both the above-kth and the equal-to-kth parts of every merge stay in token order.
    Pinned here by the literal buffer restatement on tie-heavy random rows (TopK counts
    aligned and not aligned to 256, rows ending inside and on trunk boundaries), and at
    the reference's sizes (TopK 2048, trunks 8192 and 16384)."""
    rng = np.random.default_rng(seed)
    for _ in range(40):
        topk = int(rng.choice([256, 300, 512]))
        trunk = int(rng.choice([512, 768, 1024, 2048]))
        if trunk < topk:
            continue
        valid = int(rng.integers(topk, 6 * trunk + 1))
        if rng.random() < 0.2:
            valid = trunk * int(rng.integers(1, 6))
        levels = int(rng.choice([2, 4, 40, 3000]))
        keys = rng.integers(1, levels + 1, valid + 64).astype(np.uint16)
        want = _literal_trunk_topk(keys, valid, topk, trunk)
        assert np.array_equal(ref.topk_reference(keys, valid, topk, trunk=trunk), want)
        assert np.array_equal(ref.topk_reference(keys, valid, topk), want)
    for valid, trunk in ((32768, 8192), (20000, 16384), (131072, 16384), (57344, 8192)):
        keys = rng.integers(0x8000, 0x8000 + int(rng.choice([60, 5000])), valid).astype(np.uint16)
        want = _literal_trunk_topk(keys, valid, 2048, trunk)
        assert np.array_equal(ref.topk_reference(keys, valid, trunk=trunk), want)
        assert np.array_equal(ref.topk_reference(keys, valid), want)


def test_topk_brute_force_tiny():
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(5, 40))
        k = int(rng.integers(1, n + 1))
        keys = rng.integers(0, 4, n).astype(np.uint16)
        got = ref.topk_reference(keys, n, topk=k)
        # brute force: every pair in the chosen set beats every pair outside it.
        chosen = set(got.tolist())
        assert len(chosen) == k
        for a in chosen:
            for b in set(range(n)) - chosen:
                assert (keys[a], -a) > (keys[b], -b)


def test_validate_topk_band():
    rng = np.random.default_rng(1)
    scores = rng.standard_normal(10000).astype(np.float32)
    keys = ref.sortable_key(ref.bf16_round_half_away(scores))
    sel = ref.topk_reference(keys, 10000)
    assert ref.validate_topk_band(sel, ref.score_values(keys))
    bad = sel.copy()
    bad[0] = int(np.argmin(scores))
    assert not ref.validate_topk_band(bad, ref.score_values(keys))


# ---------------------------------------------------------------- Fetch
def test_fetch_gather_known_answer():
    kv = np.stack([ref.identity_rows(np.arange(128) + 1000 * blk, 32) for blk in range(3)])
    table = np.array([[2, 0], [1, 2]], np.int32)
    topk = np.array([[0, 130, -1], [127, 5, 128]])
    out = ref.fetch_gather(kv, table, topk)
    assert np.array_equal(out[0, 0], kv[2, 0]) and np.array_equal(out[0, 1], kv[0, 2])
    assert not out[0, 2].any()
    assert np.array_equal(out[1, 0], kv[1, 127]) and np.array_equal(out[1, 2], kv[2, 0])
    rows = ref.identity_rows(np.arange(4096))
    assert len({r.tobytes() for r in rows}) == 4096


def test_prefill_visibility_closed_form():
    """Right-down causal: the last row of a sequence sees every key, rows above it one
    fewer each; a sequence with more queries than keys starts with empty rows."""
    from oracle.indexer import prefill_visible

    vis = prefill_visible(np.array([0, 4, 7]), np.array([10, 2]))
    assert vis.tolist() == [7, 8, 9, 10, 0, 1, 2]


def test_prefill_keys_equal_per_row_decode_keys():
    """Each prefill row scores the same keys as a decode row bounded at its visibility."""
    from oracle import indexer as ref

    rng = np.random.default_rng(8)
    heads, blocks = 8, 6
    keys = ref.fp8_e4m3_decode(rng.integers(0, 256, (blocks, 128, 128), dtype=np.uint8) & 0x77)
    key_scale = rng.uniform(0.5, 2, (blocks, 128)).astype(np.float32)
    query = ref.fp8_e4m3_decode(rng.integers(0, 256, (5, heads, 128), dtype=np.uint8) & 0x77)
    weights = rng.standard_normal((5, heads)).astype(np.float32) / 8
    table = np.array([[3, 1, 5], [0, 2, 4]], np.int32)
    cu, kl = np.array([0, 3, 5]), np.array([300, 257])
    got, vis = ref.prefill_keys_paged(query, weights, None, keys, key_scale, table, cu, kl, 384)
    for r, v in enumerate(vis):
        s = 0 if r < 3 else 1
        want, _ = ref.decode_keys_paged(query[r:r + 1], weights[r:r + 1], None, keys, key_scale, table[s:s + 1],
                                        [kl[s]], query_ends=[v], key_stride=384)
        assert np.array_equal(got[r], want[0]), r
