"""Pins the CPU oracle against checks that do not restate its formulas.

* the reference's closed-form LightningIndexer case, score == token id
  (ut_ops/test_fused_li_manage.py:146-173, expected top-2048 = the last 2048
  ids, :285-293), and its structured cache state (:196-216);
* brute-force Python loops on tiny inputs;
* the reference's behavioural invariants for LIM (test_fused_li_manage.py:314-426,
  FUSED_LI_MANAGE_BEHAVIOR.md:15-25) and MTP LIM (test_fused_li_manage_mtp.py:789-960);
* a library routine: attention vs torch's scaled_dot_product_attention in float64;
* special cases with a known answer (one key, equal logits, masked keys).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

TOPK = O.TOPK


# --------------------------------------------------------------------------
# 16-bit codecs
def test_bf16_codec_known_values():
    vals = np.array([1.0, -2.0, 0.5, 3.140625, 65280.0, -0.0], dtype=np.float32)
    bits = O.f32_to_bits(vals, "bf16")
    assert bits.tolist() == [0x3F80, 0xC000, 0x3F00, 0x4049, 0x477F, 0x8000]
    assert np.array_equal(O.bits_to_f32(bits, "bf16"), vals)
    # round to nearest even: 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> 1
    assert O.f32_to_bits(np.float32(1 + 2 ** -8), "bf16")[0] == 0x3F80
    assert O.f32_to_bits(np.float32(1 + 3 * 2 ** -8), "bf16")[0] == 0x3F82
    t = torch.tensor([1.7, -0.3, 1e-3, 12345.0]).to(torch.bfloat16)
    assert np.array_equal(O.f32_to_bits(t.float().numpy()), t.view(torch.int16).numpy().view(np.uint16))


def test_f16_codec_matches_numpy():
    x = np.array([0.1, -7.5, 1024.25, 3e-5], dtype=np.float32)
    assert np.array_equal(O.bits_to_f32(O.f32_to_bits(x, "f16"), "f16"), x.astype(np.float16).astype(np.float32))


# --------------------------------------------------------------------------
# scores
def _digit_keys(ids: np.ndarray) -> np.ndarray:
    k = np.zeros((ids.size, 128), dtype=np.float32)
    k[:, 0] = ids % 64
    k[:, 1] = (ids // 64) % 64
    k[:, 2] = (ids // 4096) % 64
    k[:, 3] = ids // 262144
    return k


def _digit_query(heads: int) -> tuple[np.ndarray, np.ndarray]:
    q = np.zeros((heads, 128), dtype=np.float32)
    q[0, :4] = [1, 64, 4096, 262144]
    w = np.zeros(heads, dtype=np.float32)
    w[0] = 1
    return q, w


def test_scores_closed_form_token_id():
    ids = np.array([0, 1, 63, 64, 4095, 4096, (1 << 18) - 1, 1 << 18, (7 << 18) + 12345, (1 << 21) - 2])
    q, w = _digit_query(32)
    s = O.index_scores(q, w, _digit_keys(ids))
    assert np.array_equal(s, ids.astype(np.float64))


def test_scores_brute_force_loops():
    rng = np.random.default_rng(3)
    H, T = 3, 5
    q = rng.standard_normal((H, 128))
    w = rng.uniform(0, 1, H)
    k = rng.standard_normal((T, 128))
    expect = []
    for t in range(T):
        tot = 0.0
        for h in range(H):
            dot = 0.0
            for d in range(128):
                dot += q[h][d] * k[t][d]
            tot += w[h] * (dot if dot > 0 else 0.0)
        expect.append(tot)
    assert np.allclose(O.index_scores(q, w, k), expect, rtol=1e-12, atol=1e-12)


def test_scores_relu_and_weights_hand_example():
    q = np.zeros((2, 128))
    q[0, 0] = 1.0
    q[1, 0] = -1.0
    k = np.zeros((1, 128))
    k[0, 0] = 2.0
    w = np.array([0.5, 3.0])
    # 0.5 * relu(2) + 3 * relu(-2) = 1
    assert O.index_scores(q, w, k)[0] == 1.0


def test_gather_rows_follows_block_table():
    cache = np.arange(3 * 128 * 2).reshape(3, 128, 1, 2)
    table = np.array([2, 0])
    rows = O.gather_rows(cache, table, 130)
    assert np.array_equal(rows[0], cache[2, 0, 0])
    assert np.array_equal(rows[127], cache[2, 127, 0])
    assert np.array_equal(rows[128], cache[0, 0, 0])
    assert np.array_equal(rows[129], cache[0, 1, 0])


def test_paged_scores_unmapped_blocks():
    """Tokens of a block-table entry that names no block score -FLT_MAX;
    the rest equal the brute-force scores of the rows the entry names."""
    rng = np.random.default_rng(2)
    cache = rng.standard_normal((4, 128, 1, 8))
    q = rng.standard_normal((3, 8))
    w = rng.standard_normal(3)
    table = np.array([3, -1, 1, 4, 0, 2])  # -1 and 4 (== block count) name no block
    n = 5 * 128 + 17
    s = O.index_scores_paged(q, w, cache, table, n)
    flt_max = float(np.finfo(np.float32).max)
    for t in range(n):
        phys = table[t // 128]
        if phys < 0 or phys >= 4:
            assert s[t] == -flt_max
        else:
            k = cache[phys, t % 128, 0]
            assert np.isclose(s[t], sum(w[h] * max(0.0, float(q[h] @ k)) for h in range(3)), rtol=1e-12, atol=1e-12)


def test_unmapped_block_tokens_rank_after_free_slots_before_scored():
    # n = 2300, C = 2049: two misses.  Slots 0..2045 hold hits; slot 2048 is
    # free; token 0 (slot 2047) sits in an unmapped block (-FLT_MAX); token
    # 128 (slot 2046) scores 0.  Victims: the free slot and token 0's slot.
    n, c = 2300, 2049
    scores = np.arange(n, dtype=np.float64)
    scores[:128] = -float(np.finfo(np.float32).max)  # block 0 unmapped
    scores[128] = 0.0
    row = np.full(n, -1, np.int64)
    top = np.arange(n - TOPK, n)
    row[top[2:]] = np.arange(TOPK - 2)
    row[128] = 2046
    row[0] = 2047
    src, dst, m = O.lim_manage_row(scores, row, n, c)
    assert m == 2 and src[:2].tolist() == top[:2].tolist()
    assert dst[:2].tolist() == [2047, 2048]
    assert row[0] == -1 and row[128] == 2046


# --------------------------------------------------------------------------
# top-k
def test_topk_closed_form_last_ids():
    n = 5000
    mask = O.topk_mask(np.arange(n, dtype=np.float64), TOPK)
    assert np.array_equal(np.nonzero(mask)[0], np.arange(n - TOPK, n))


def test_topk_ties_lower_index_and_brute_force():
    rng = np.random.default_rng(5)
    for trial in range(5):
        n, k = 40, 13
        s = rng.integers(0, 6, n).astype(np.float64)
        expect = sorted(range(n), key=lambda i: (-s[i], i))[:k]
        mask = O.topk_mask(s, k)
        assert sorted(np.nonzero(mask)[0].tolist()) == sorted(expect)
    assert np.array_equal(np.nonzero(O.topk_mask(np.zeros(10), 4))[0], [0, 1, 2, 3])


# --------------------------------------------------------------------------
# LIM bookkeeping (MTP0)
def _structured_state(seq_len, cache_tokens, miss_count, seed, pool_rows=2, row=1):
    """The reference's structured cache state (test_fused_li_manage.py:196-216):
    score == id, hits = top-k[miss:], the rest spread evenly below."""
    topk = np.arange(seq_len - TOPK, seq_len)
    hit_tokens = topk[miss_count:]
    other_count = cache_tokens - hit_tokens.size
    lower = seq_len - TOPK
    others = (np.arange(other_count) * lower) // other_count if other_count else np.zeros(0, np.int64)
    cached = np.concatenate([hit_tokens, others])
    pool = np.full((pool_rows, seq_len), -1, dtype=np.int64)
    rng = np.random.default_rng(seed)
    pool[row, cached] = rng.permutation(cache_tokens)
    return pool, cached, others


def _check_lim_invariants(src, dst, m, old_row, new_row, scores, n, c, expected_miss):
    """Port of validate_outputs (test_fused_li_manage.py:314-426)."""
    assert m == expected_miss
    assert np.unique(src).size == TOPK and src.min() >= 0 and src.max() < n
    expect_set = np.nonzero(O.topk_mask(scores, TOPK))[0]
    assert np.array_equal(np.sort(src), expect_set)
    assert dst.min() >= 0 and dst.max() < c and np.unique(dst).size == TOPK
    old = old_row[src]
    miss_mask = old == -1
    assert miss_mask.sum() == expected_miss
    assert miss_mask[:m].all() and not miss_mask[m:].any()  # miss prefix / hit suffix
    assert np.array_equal(dst[m:], old[m:])  # hit slots preserved
    assert np.array_equal(new_row[src], dst)  # itemwise map
    for state in (old_row, new_row):
        valid = state[state >= 0]
        assert valid.size == c and np.unique(valid).size == c and valid.min() == 0 and valid.max() == c - 1


@pytest.mark.parametrize("seq_len,cache_tokens,miss", [(4096, 2048, 300), (6144, 3072, 200), (8192, 4096, 0),
                                                        (2048 + 1280, 2560, 640)])
def test_lim_structured_invariants_and_repeat(seq_len, cache_tokens, miss):
    pool, cached, others = _structured_state(seq_len, cache_tokens, miss, seed=7)
    before = pool.copy()
    scores = np.arange(seq_len, dtype=np.float64)
    src, dst, m = O.lim_manage_row(scores, pool[1], seq_len, cache_tokens)
    _check_lim_invariants(src, dst, m, before[1], pool[1], scores, seq_len, cache_tokens, miss)
    assert np.array_equal(pool[0], before[0])  # unmapped pool row unchanged
    # canonical order: misses ascending, hits by descending old slot
    assert np.array_equal(src[:m], np.arange(seq_len - TOPK, seq_len - TOPK + miss))
    assert np.all(np.diff(dst[m:]) < 0)
    # victims: the m lowest-score cached non-selected tokens (score == id)
    victims = np.sort(others)[:m]
    assert np.all(pool[1][victims] == -1)
    assert np.array_equal(np.sort(before[1][victims]), dst[:m])  # paired ascending
    # a second update with the same query sees zero misses
    second = pool.copy()
    src2, dst2, m2 = O.lim_manage_row(scores, pool[1], seq_len, cache_tokens)
    _check_lim_invariants(src2, dst2, m2, second[1], pool[1], scores, seq_len, cache_tokens, 0)


def test_lim_forced_victims_when_c_is_2048():
    rng = np.random.default_rng(11)
    n, c = 4096, 2048
    scores = rng.permutation(n).astype(np.float64)
    sel = O.topk_mask(scores, TOPK)
    sel_ids = np.nonzero(sel)[0]
    hits = rng.choice(sel_ids, 1800, replace=False)
    others = rng.choice(np.nonzero(~sel)[0], c - hits.size, replace=False)
    row = np.full(n, -1, np.int64)
    row[np.concatenate([hits, others])] = rng.permutation(c)
    old = row.copy()
    src, dst, m = O.lim_manage_row(scores, row, n, c)
    assert m == TOPK - hits.size
    assert np.all(row[others] == -1)  # every cached unselected token is evicted
    assert np.array_equal(dst[:m], np.sort(old[others]))
    _check_lim_invariants(src, dst, m, old, row, scores, n, c, m)


def test_lim_hand_example_small_tie_rules():
    # n = 2052, C = 2049: scores make tokens 0..3 the four lowest.
    n, c = 2052, 2049
    scores = np.arange(n, dtype=np.float64)
    scores[2] = scores[3] = 0.5  # tie between cached candidates 2 and 3
    # cached: 0 (slot 7), 2 (slot 5), 3 (slot 9), and all top tokens except 4 and 5 (misses)
    row = np.full(n, -1, np.int64)
    top = np.arange(4, n)  # the 2048 selected tokens
    hits = top[2:]  # tokens 4 and 5 miss
    slots = np.random.default_rng(0).permutation(c)
    cached = np.concatenate([[0, 2, 3], hits])
    row[cached] = slots
    old = row.copy()
    src, dst, m = O.lim_manage_row(scores, row, n, c)
    assert m == 2 and src[:2].tolist() == [4, 5]
    # candidates 0 (0.0), 2 (0.5), 3 (0.5): victims = token 0 and, on the tie,
    # the lower slot of tokens 2/3
    tie_winner = 2 if old[2] < old[3] else 3
    victim_slots = sorted([old[0], old[tie_winner]])
    assert dst[:2].tolist() == victim_slots
    assert row[0] == -1 and row[tie_winner] == -1 and row[5 - tie_winner] == old[5 - tie_winner]
    assert row[4] == victim_slots[0] and row[5] == victim_slots[1]


def test_lim_free_slots_are_used_first():
    n, c = 2100, 2050
    scores = np.arange(n, dtype=np.float64)
    row = np.full(n, -1, np.int64)
    # 2047 of the top tokens cached on slots 0..2046; token 0 cached on 2047;
    # slots 2048, 2049 held by nobody; token n-1 (selected) misses.
    top = np.arange(n - TOPK, n)
    row[top[:-1]] = np.arange(TOPK - 1)
    row[0] = TOPK - 1
    src, dst, m = O.lim_manage_row(scores, row, n, c)
    assert m == 1 and src[0] == n - 1 and dst[0] == 2048  # lowest free slot
    assert row[0] == TOPK - 1  # the candidate keeps its slot


def test_lim_guards_write_zero_miss_and_touch_nothing():
    B = 6
    n_list = [0, 4096, 4096, 4096, 1000, 4096]
    c_list = [2048, 0, 1024, 5000, 2048, 2048]
    r_list = [0, 1, 2, 3, 4, 9]  # last row index out of range
    pool = np.full((5, 4096), -1, np.int32)
    before = pool.copy()
    q = np.zeros((B, 32, 128), np.uint16)
    w = np.zeros((B, 32), np.uint16)
    kc = np.zeros((32, 128, 1, 128), np.uint16)
    table = np.zeros((B, 32), np.int32)
    src = np.full((B, 1, TOPK), 9, np.int32)
    dst = np.full((B, 1, TOPK), 9, np.int32)
    mc = np.full(B, 9, np.int32)
    O.fused_li_manage(q, w, kc, table, np.array(n_list), np.array(c_list), np.array(r_list), pool, src, dst, mc)
    assert mc.tolist() == [0] * B
    assert np.array_equal(pool, before)
    assert np.all(src == 9) and np.all(dst == 9)


# --------------------------------------------------------------------------
# MTP3 LIM
def test_ordered_union_definition():
    rows = [np.array([5, 1, 9]), np.array([1, 2]), np.array([9, 7, 2]), np.array([3])]
    assert O.ordered_union(rows).tolist() == [5, 1, 9, 2, 7, 3]


def test_mtp_invariants_random():
    rng = np.random.default_rng(21)
    n, c = 9000, 8192
    base = rng.standard_normal(n)
    scores4 = np.stack([base + 0.3 * rng.standard_normal(n) for _ in range(4)])
    rows = [np.nonzero(O.topk_mask(scores4[q], TOPK))[0] for q in range(4)]
    union = O.ordered_union(rows)
    miss = rng.choice(union, 150, replace=False)
    hits = np.setdiff1d(union, miss)
    fill = rng.choice(np.setdiff1d(np.arange(n), union), c - hits.size, replace=False)
    pool_row = np.full(n, -1, np.int64)
    pool_row[np.concatenate([hits, fill])] = rng.permutation(c)
    before = pool_row.copy()
    rs, rd, ms, md = O.lim_manage_mtp_row(scores4, pool_row, n, c)
    after = pool_row
    # port of validate_result (test_fused_li_manage_mtp.py:789-960)
    valid = after[after >= 0]
    assert valid.size == c and np.unique(valid).size == c
    cached_tokens = np.nonzero(after >= 0)[0]
    slot_to_token = np.full(c, -1)
    slot_to_token[after[cached_tokens]] = cached_tokens
    actual_rows = []
    for q in range(4):
        s = rd[q].astype(np.int64)
        assert s.min() >= 0 and s.max() < c and np.unique(s).size == TOPK
        toks = slot_to_token[s]
        assert np.array_equal(rs[q], np.where(before[toks] < 0, toks, -1))
        assert np.array_equal(np.sort(toks), rows[q])
        assert np.array_equal(toks, rows[q])  # canonical row order: ascending token id
        actual_rows.append(toks)
    u = O.ordered_union(actual_rows)
    assert np.array_equal(u, union)
    assert np.all(after[union] >= 0)
    expected_misses = union[before[union] < 0]
    assert np.array_equal(ms, expected_misses) and ms.size == 150
    assert np.unique(md).size == md.size and md.min() >= 0 and md.max() < c
    old_hits = union[before[union] >= 0]
    assert np.array_equal(after[old_hits], before[old_hits])
    assert np.array_equal(after[expected_misses], md)
    old_tokens = np.nonzero(before >= 0)[0]
    evicted = old_tokens[after[old_tokens] < 0]
    assert not np.isin(evicted, union).any()
    # victims are the lowest max-score fillers
    smax = scores4.max(axis=0)
    assert np.array_equal(np.sort(evicted), np.sort(fill[np.argsort(smax[fill], kind="stable")[:150]]))


# --------------------------------------------------------------------------
# scatter_copy
def test_scatter_copy_rules():
    rng = np.random.default_rng(2)
    B, cap = 3, 16
    dram_kpe = rng.integers(0, 65535, (6, 128, 64), dtype=np.uint16)
    dram_ckv = rng.integers(0, 65535, (6, 128, 512), dtype=np.uint16)
    hbm_kpe = rng.integers(0, 65535, (4, 128, 64), dtype=np.uint16)
    hbm_ckv = rng.integers(0, 65535, (4, 128, 512), dtype=np.uint16)
    dram_table = np.array([[0, 1], [2, 3], [4, -1]], np.int32)
    hbm_table = np.array([[0], [1], [2]], np.int32)
    src = np.full((B, cap), -1, np.int32)
    dst = np.full((B, cap), -1, np.int32)
    src[0, :3] = [5, 200, 7]
    dst[0, :3] = [1, 2, -4]          # third pair skipped (negative slot)
    src[1, :2] = [130, 3]
    dst[1, :2] = [127, 500]          # second pair skipped (slot beyond table)
    src[2, :2] = [140, 1]
    dst[2, :2] = [3, 4]              # first pair skipped (dram column -1)
    counts = np.array([3, 2, 99], np.int32)  # 99 clamps to cap
    h0k, h0c = hbm_kpe.copy(), hbm_ckv.copy()
    O.scatter_copy(src, dst, counts, hbm_table, dram_table, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv)
    expect_c, expect_k = h0c.copy(), h0k.copy()
    for (hb, ho, db, do) in [(0, 1, 0, 5), (0, 2, 1, 72), (1, 127, 3, 2), (2, 4, 4, 1)]:
        expect_c[hb, ho] = dram_ckv[db, do]
        expect_k[hb, ho] = dram_kpe[db, do]
    assert np.array_equal(hbm_ckv, expect_c) and np.array_equal(hbm_kpe, expect_k)


# --------------------------------------------------------------------------
# attention
def _attn_case(rng, cases, heads=4, rows_per_request=1):
    B = len(cases)
    lens = [c + t for c, t in cases]
    cols = max(1, math.ceil(max(lens) / 128))
    table = rng.permutation(B * cols).reshape(B, cols).astype(np.int32)
    ckv = O.f32_to_bits(0.25 * rng.standard_normal((B * cols, 128, 1, 512)).astype(np.float32))
    kpe = O.f32_to_bits(0.25 * rng.standard_normal((B * cols, 128, 1, 64)).astype(np.float32))
    R = B * rows_per_request
    q = O.f32_to_bits(0.25 * rng.standard_normal((R, heads, 512)).astype(np.float32))
    qr = O.f32_to_bits(0.25 * rng.standard_normal((R, heads, 64)).astype(np.float32))
    topk = np.zeros((R, 1, TOPK), np.int32)
    for r in range(R):
        c = cases[r // rows_per_request][0]
        if c >= TOPK:
            topk[r, 0] = rng.permutation(c)[:TOPK]
    return dict(query_rope=qr, query=q, seq_kv=np.array(lens), num_cache=np.array([c for c, _ in cases]),
                topk_dst=topk, hbm_table=table, hbm_kpe=kpe, hbm_ckv=ckv)


def test_attention_matches_torch_sdpa_float64():
    rng = np.random.default_rng(4)
    cases = [(0, 1), (0, 129), (2048, 0), (3072, 257)]
    a = _attn_case(rng, cases)
    scale = 1 / math.sqrt(576)
    out = O.sparse_tail_attention(**a, scale=scale)
    ckv = O.bits_to_f32(a["hbm_ckv"]).reshape(-1, 512).astype(np.float64)
    kpe = O.bits_to_f32(a["hbm_kpe"]).reshape(-1, 64).astype(np.float64)
    for b, (c, t) in enumerate(cases):
        slots = np.arange(t) if c == 0 else np.concatenate([a["topk_dst"][b, 0], np.arange(c, c + t)])
        phys = a["hbm_table"][b, slots // 128].astype(np.int64) * 128 + slots % 128
        qq = np.concatenate([O.bits_to_f32(a["query"][b]), O.bits_to_f32(a["query_rope"][b])], -1)
        kk = np.concatenate([ckv[phys], kpe[phys]], -1)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(qq.astype(np.float64))[:, None], torch.from_numpy(kk)[None].expand(qq.shape[0], -1, -1),
            torch.from_numpy(ckv[phys])[None].expand(qq.shape[0], -1, -1), scale=scale)
        assert np.allclose(out[b], ref[:, 0].numpy(), rtol=1e-10, atol=1e-12)


def test_attention_special_cases():
    rng = np.random.default_rng(8)
    # a single visible key: output == that key's ckv row
    a = _attn_case(rng, [(0, 1)])
    out = O.sparse_tail_attention(**a, scale=0.1)
    row0 = O.bits_to_f32(a["hbm_ckv"])[a["hbm_table"][0, 0], 0, 0]
    assert np.allclose(out[0], np.broadcast_to(row0, out[0].shape))
    # zero query: uniform softmax -> mean of the visible rows
    a = _attn_case(rng, [(0, 300)])
    a["query"][:] = 0
    a["query_rope"][:] = 0
    out = O.sparse_tail_attention(**a, scale=0.1)
    rows = O.gather_rows(O.bits_to_f32(a["hbm_ckv"]), a["hbm_table"][0], 300)
    assert np.allclose(out[0], rows.mean(0), atol=1e-6)
    # inactive rows (0 < C < 2048, C > L) -> zeros
    a = _attn_case(rng, [(1024, 5), (2048, 0)])
    a["seq_kv"][1] = 2000  # C = 2048 > L
    out = O.sparse_tail_attention(**a, scale=0.1)
    assert np.all(out == 0)


def test_attention_mtp_causal_visible_length():
    rng = np.random.default_rng(9)
    c, t = 2048, 10
    a = _attn_case(rng, [(c, t)], rows_per_request=4)
    out = O.sparse_tail_attention(**a, scale=1 / 24, rows_per_request=4)
    for q in range(4):
        vis = c + t - (3 - q)
        one = {k: (v[q:q + 1] if k in ("query", "query_rope", "topk_dst") else v) for k, v in a.items()}
        one["seq_kv"] = np.array([vis])
        ref = O.sparse_tail_attention(**one, scale=1 / 24, rows_per_request=1)
        assert np.allclose(out[q], ref[0])
    # query 0 must not see the last three tail tokens: make them dominant
    a2 = {k: v.copy() for k, v in a.items()}
    ckv = a2["hbm_ckv"].reshape(-1, 512)
    for s in range(c + t - 3, c + t):
        prow = a2["hbm_table"][0, s // 128] * 128 + s % 128
        ckv[prow] = O.f32_to_bits(np.full(512, 50.0, np.float32))
    out2 = O.sparse_tail_attention(**a2, scale=1 / 24, rows_per_request=4)
    assert np.allclose(out2[0], out[0])
    assert not np.allclose(out2[3], out[3])


# --------------------------------------------------------------------------
# prefill -> DRAM hand-over
def test_persist_blocks_brute_force():
    rng = np.random.default_rng(11)
    hbm_ckv = rng.integers(0, 1 << 16, (5, 128, 1, 8), dtype=np.uint16)
    hbm_kpe = rng.integers(0, 1 << 16, (5, 128, 1, 2), dtype=np.uint16)
    dram_ckv = rng.integers(0, 1 << 16, (7, 128, 1, 8), dtype=np.uint16)
    dram_kpe = rng.integers(0, 1 << 16, (7, 128, 1, 2), dtype=np.uint16)
    before_c, before_k = dram_ckv.copy(), dram_kpe.copy()
    hbm_ids = np.array([4, 0, -1, 2, 9], np.int32)
    dram_ids = np.array([1, 6, 3, 7, 2], np.int32)  # pairs 3 (dram 7) and 4 (hbm 9) and 2 (hbm -1) are skipped
    O.persist_blocks(hbm_ckv, hbm_kpe, dram_ckv, dram_kpe, hbm_ids, dram_ids)
    for d in range(7):
        for t in range(128):
            for e in range(8):
                want = {1: hbm_ckv[4], 6: hbm_ckv[0]}.get(d, before_c[d])[t, 0, e]
                assert dram_ckv[d, t, 0, e] == want
            for e in range(2):
                want = {1: hbm_kpe[4], 6: hbm_kpe[0]}.get(d, before_k[d])[t, 0, e]
                assert dram_kpe[d, t, 0, e] == want


def test_finalize_prefill_pool_row_branches():
    row = np.full(1024, 7, np.int32)
    # long request: reset only, persist
    assert O.finalize_prefill_pool_row(row, num_full_blocks=5, num_sparse_blocks=2, cache_tokens=2048)
    assert (row == -1).all()
    # short request with a budget: identity over the full blocks
    row[:] = 7
    assert not O.finalize_prefill_pool_row(row, num_full_blocks=3, num_sparse_blocks=3, cache_tokens=2048)
    assert np.array_equal(row[:384], np.arange(384)) and (row[384:] == -1).all()
    # short request, no budget: reset only
    row[:] = 7
    assert not O.finalize_prefill_pool_row(row, num_full_blocks=3, num_sparse_blocks=4, cache_tokens=0)
    assert (row == -1).all()
    # shared (non-owner) layer: the row is not touched
    row[:] = 7
    assert O.finalize_prefill_pool_row(row, num_full_blocks=5, num_sparse_blocks=2, cache_tokens=2048, owner=False)
    assert (row == 7).all()

