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
