"""The seeded workload generator builds consistent, margin-guarded inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, ints, oracle_lim
from oracle import dsa_oracle as O


@pytest.mark.parametrize("mtp", [False, True])
def test_generator_state_is_consistent(mtp):
    from nanovllm_amd.workloads import make_chain_case

    if mtp:
        case = make_chain_case(2, [9216, 10240], [8192, 8448], [4, 9], seed=3, mtp=True)
    else:
        case = make_chain_case(3, [4096, 6144, 4096], [2048, 3072, 0], [5, 9, 100], seed=3)
    t = case.tensors
    pool = ints(t["cache_slots_pool"])
    entries = ints(t["req_pool_entries"])
    hc = bits(t["hbm_kv_cache"]).reshape(-1, 512)
    dc = bits(t["dram_kv_cache"]).reshape(-1, 512)
    for b in range(case.meta["batch"]):
        c = case.meta["cache_tokens"][b]
        row = pool[entries[b]]
        valid = row[row >= 0]
        assert valid.size == c and np.unique(valid).size == c
        for tok in np.nonzero(row >= 0)[0][:50]:
            s = row[tok]
            hrow = ints(t["hbm_block_table"])[b, s // 128] * 128 + s % 128
            drow = ints(t["dram_block_table"])[b, tok // 128] * 128 + tok % 128
            assert np.array_equal(hc[hrow], dc[drow])
    unmapped = [r for r in range(pool.shape[0]) if r not in entries.tolist()]
    assert all(np.all(pool[r] == -777) for r in unmapped)


def test_generator_miss_rate_and_margins():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(2, [8192, 8192], [2048, 4096], [1, 2], seed=17)
    exp = oracle_lim(case)
    for b in range(2):
        m = exp["miss_counts"][b]
        assert m == case.meta["miss_target"][b]
        assert 0.05 * 2048 - 1 <= m <= 0.15 * 2048 + 1
    # top-k boundary gap exceeds the fp32 reduction-order bound
    t = case.tensors
    kc = O.bits_to_f32(bits(t["index_key_cache"]))
    for b in range(2):
        keys = O.gather_rows(kc, ints(t["index_block_table"])[b], 8192).astype(np.float64)
        q = O.bits_to_f32(bits(t["query_index"]))[b].astype(np.float64)
        w = O.bits_to_f32(bits(t["index_weights"]))[b].astype(np.float64)
        s = O.index_scores(q, w, keys)
        e = 2.0 ** -24 * 256 * (np.abs(keys) @ np.abs(q).T) @ np.abs(w)
        order = np.lexsort((np.arange(s.size), -s))
        a, z = order[2047], order[2048]
        assert s[a] - s[z] >= e[a] + e[z]


def test_drift_guard_makes_every_step_order_independent():
    """``make_drift_case(guard=True)`` pins every step of the alternating
    sequence: moving each step's float64 scores anywhere within their fp32
    reduction-error bounds leaves every step's ids, slots, miss counts and the
    carried pool unchanged (the property the GPU carried-state test relies
    on).  Cache budgets above 2048 make the victims depend on the scores and
    on the cached set the earlier steps left."""
    from nanovllm_amd.workloads import make_drift_case

    steps = 5
    case = make_drift_case(3, [8192, 12288, 6144], [2048, 3072, 2560], [5, 9, 100], seed=5, guard=True,
                           guard_steps=steps, guard_first="query_index", miss_frac=(0.1, 0.2))
    t = case.tensors
    kc = O.bits_to_f32(bits(t["index_key_cache"])).astype(np.float64)
    w = O.bits_to_f32(bits(t["index_weights"])).astype(np.float64)
    table = ints(t["index_block_table"])
    entries = ints(t["req_pool_entries"])
    rng = np.random.default_rng(99)
    names = ("query_index", "query_index_b")
    exact = ints(t["cache_slots_pool"])
    moved = exact.copy()
    misses = []
    for step in range(steps):
        q = O.bits_to_f32(bits(t[names[step % 2]])).astype(np.float64)
        total = 0
        for b in range(case.meta["batch"]):
            n, c = case.meta["source_lens"][b], case.meta["cache_tokens"][b]
            keys = O.gather_rows(kc, table[b], n)
            s = O.index_scores(q[b], w[b], keys)
            e = 2.0 ** -24 * 256 * (np.abs(keys) @ np.abs(q[b]).T) @ np.abs(w[b])
            noisy = s + e * rng.uniform(-0.999, 0.999, size=s.shape)
            r = entries[b]
            got = O.lim_manage_row(noisy, moved[r], n, c)
            want = O.lim_manage_row(s, exact[r], n, c)
            for x, y in zip(got, want):
                assert np.array_equal(np.asarray(x), np.asarray(y)), (step, b)
            assert np.array_equal(moved[r], exact[r]), (step, b)
            total += want[2]
        misses.append(total)
    assert min(misses[1:]) > 0, misses


def test_structured_drift_scores_are_exact_and_keep_missing():
    """``make_structured_drift_case``: every row's fp32 scores (torch's own
    summation order) equal the float64 integers exactly, the rows select
    different sets, and alternating the two queries keeps producing misses
    with C = 8192 (victims chosen by score over the carried cached set)."""
    from nanovllm_amd.workloads import make_structured_drift_case

    orders_a = [(1.0, 64.0, 4096.0, 0.0), (4096.0, 1.0, 64.0, 0.0), (1.0, 4096.0, 64.0, 0.0), (64.0, 4096.0, 1.0, 0.0)]
    orders_b = [(64.0, 1.0, 4096.0, 0.0), (64.0, 4096.0, 1.0, 0.0), (4096.0, 64.0, 1.0, 0.0), (1.0, 4096.0, 64.0, 0.0)]
    case = make_structured_drift_case(2, [49152, 40960], [8192, 8192], [4, 9], orders_a, orders_b, seed=3)
    t = case.tensors
    kc = t["index_key_cache"].view(-1, 128)
    table = t["index_block_table"]
    for name in ("query_index", "query_index_b"):
        for b in range(2):
            n = case.meta["source_lens"][b]
            tok = torch.arange(n)
            keys = kc[table[b, tok // 128].long() * 128 + tok % 128]
            for j in range(4):
                q, w = t[name][4 * b + j], t["index_weights"][4 * b + j]
                s32 = torch.relu(keys.float() @ q.float().T) @ w.float()
                s64 = torch.relu(keys.double() @ q.double().T) @ w.double()
                assert torch.equal(s32.double(), s64), (name, b, j)
                assert torch.equal(s64, torch.round(s64)) and np.unique(s64.numpy()).size == n
    pool = ints(t["cache_slots_pool"])
    R = 8
    misses = []
    for name in ("query_index", "query_index", "query_index_b", "query_index", "query_index_b"):
        src = np.zeros((R, 1, 2048), np.int32)
        dst = np.zeros((R, 1, 2048), np.int32)
        ms = np.zeros((2, 8192), np.int32)
        md = np.zeros((2, 8192), np.int32)
        mc = np.zeros(2, np.int32)
        O.fused_li_manage_mtp(bits(t[name]), bits(t["index_weights"]), bits(t["index_key_cache"]),
                              ints(t["index_block_table"]), ints(t["num_candidate_tokens"]),
                              ints(t["num_cache_tokens"]), ints(t["req_pool_entries"]), pool, src, dst, ms, md, mc)
        misses.append(mc.tolist())
    assert misses[1] == [0, 0] and all(min(m) > 0 for m in misses[2:]), misses
