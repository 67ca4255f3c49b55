"""The reference's own LIM / attention cases that stress layouts the random
tests do not reach, on the GPU vs the oracle.

* Cache tiers C in {6144, 8192, 12288, 16383} with candidates <= 32768
  (ut_ops/test_fused_li_manage_scatter.py:21-23): the manage kernel that
  keeps a request's scores in registers, with slot tables too large for LDS.
  Margin-guarded random keys (top-2048 and victim boundaries); every integer
  output and the pool bit-exact, then the fused copy + attention.
* The reference's bs=24 local-schedule case (test_fused_li_manage_scatter.py:541-755):
  24 requests over the same 156 index blocks, score == token id (keys
  (id // 256, id % 256), query (256, 1)), C = 6144, 300 misses per request,
  pool rows in shuffled order.  Its invariants and the oracle bit-exact, and
  the repeat call has no misses.
* Attention with C equal to the whole source, so the selected slots are
  logical token ids past 2^14 (ut_ops/test_glm_mtp_index_share_slots.py:121-230):
  source 20992 + tail 64, HBM holding the whole sequence, MTP0 and MTP3
  rows, against the float64 golden.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _chain import check_copy_attend, check_lim, oracle_chain, poison_outputs, run_copy_attend, run_lim
from _helpers import assert_attention_close, bits, dname, ints, oracle_lim
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
TOPK = 2048


@pytest.mark.parametrize("mtp", [False, True])
def test_large_cache_tiers_on_the_register_path(mtp):
    from nanovllm_amd.workloads import make_chain_case

    if mtp:
        case = make_chain_case(3, [16384, 24576, 32768], [8192, 12288, 16383], [4, 60, 127], seed=61, mtp=True,
                               fast_fill=True)
    else:
        case = make_chain_case(4, [16384, 24576, 32768, 32768], [6144, 8192, 12288, 16383], [1, 64, 127, 30],
                               seed=62, fast_fill=True)
    assert case["cache_slots_pool"].shape[1] == 32768
    print(f"TIERS mtp={mtp} halvings={case.meta['halvings']} miss={case.meta['miss_target']}", flush=True)
    lim = oracle_lim(case, mtp=mtp)
    gold, hkpe, hckv = oracle_chain(case, lim, mtp)
    d = case.to_device("cuda").tensors
    poison_outputs(d, mtp)
    run_lim(d, mtp)
    torch.cuda.synchronize()
    check_lim(d, lim, mtp, f"tiers mtp={mtp}")
    run_copy_attend(d, case.meta["scale"], mtp, fused=True)
    torch.cuda.synchronize()
    check_copy_attend(d, gold, hkpe, hckv, f"tiers mtp={mtp}")


def _bs24_case(heads: int, seed: int = 7):
    """The reference's run_local_bs24_case inputs (test_fused_li_manage_scatter.py:548-612)."""
    from nanovllm_amd.workloads import ChainCase

    batch, n, c, miss = 24, 19968, 6144, 300
    blocks = n // 128
    g = torch.Generator().manual_seed(seed + heads + 2400)
    table = torch.arange(blocks, dtype=torch.int32).repeat(batch, 1)
    ids = torch.arange(n, dtype=torch.int64).reshape(blocks, 128)
    key = torch.zeros(blocks, 128, 1, 128)
    key[:, :, 0, 0] = (ids // 256).float()
    key[:, :, 0, 1] = (ids % 256).float()
    query = torch.zeros(batch, heads, 128)
    query[:, 0, 0] = 256
    query[:, 0, 1] = 1
    weights = torch.zeros(batch, heads)
    weights[:, 0] = 1
    entries = torch.randperm(batch, generator=g).to(torch.int32)
    pool = torch.full((batch, n), -1, dtype=torch.int32)
    kept = TOPK - miss
    cached = torch.cat((torch.arange(n - kept, n), torch.arange(c - kept)))
    for row in range(batch):
        pool[int(entries[row]), cached] = torch.randperm(c, generator=g).to(torch.int32)
    t = {
        "query_index": query.to(torch.bfloat16), "index_weights": weights.to(torch.bfloat16),
        "index_key_cache": key.to(torch.bfloat16), "index_block_table": table,
        "num_candidate_tokens": torch.full((batch,), n, dtype=torch.int32),
        "num_cache_tokens": torch.full((batch,), c, dtype=torch.int32), "req_pool_entries": entries,
        "cache_slots_pool": pool, "topk_src_ids": torch.full((batch, 1, TOPK), -5, dtype=torch.int32),
        "topk_dst_slots": torch.full((batch, 1, TOPK), -5, dtype=torch.int32),
        "miss_counts": torch.full((batch,), -5, dtype=torch.int32),
    }
    return ChainCase(t, {}), n, c, miss


@pytest.mark.parametrize("heads", [32, 64])
def test_reference_bs24_shuffled_pool_case(heads):
    case, n, c, miss = _bs24_case(heads)
    print(f"BS24 heads={heads}", flush=True)
    lim = oracle_lim(case)
    old = ints(case["cache_slots_pool"])
    d = case.to_device("cuda").tensors
    run_lim(d, False)
    torch.cuda.synchronize()
    check_lim(d, lim, False, f"bs24 heads={heads}")
    # the reference's own invariants (test_fused_li_manage_scatter.py:660-721)
    counts = ints(d["miss_counts"])
    assert (counts == miss).all(), counts
    topk = np.arange(n - TOPK, n)
    pool = ints(d["cache_slots_pool"])
    src = ints(d["topk_src_ids"]).reshape(24, TOPK).astype(np.int64)
    dst = ints(d["topk_dst_slots"]).reshape(24, TOPK).astype(np.int64)
    entries = ints(d["req_pool_entries"])
    for row in range(24):
        state = pool[entries[row]]
        valid = state[state >= 0]
        assert valid.size == c and np.unique(valid).size == c and valid.min() == 0 and valid.max() == c - 1
        assert (state[topk] >= 0).all()
        assert np.array_equal(np.sort(src[row]), topk)
        assert np.array_equal(np.sort(src[row, :miss]), topk[:miss])
        act = dst[row, :miss]
        assert (act >= 0).all() and (act < c).all() and np.unique(act).size == miss
        assert np.array_equal(np.sort(dst[row]), np.sort(state[topk]))
        assert (old[entries[row]][src[row, :miss]] < 0).all()
    # identical query again: everything is cached
    run_lim(d, False)
    torch.cuda.synchronize()
    assert (ints(d["miss_counts"]) == 0).all()
    pool2 = ints(d["cache_slots_pool"])
    assert np.array_equal(pool2, pool)
    src2 = ints(d["topk_src_ids"]).reshape(24, TOPK)
    dst2 = ints(d["topk_dst_slots"]).reshape(24, TOPK)
    for row in range(24):
        assert np.array_equal(np.sort(src2[row]), topk)
        assert np.array_equal(np.sort(dst2[row]), np.sort(pool2[entries[row]][topk]))


@pytest.mark.parametrize("rows_per_request,heads", [(1, 2), (1, 64), (4, 64)])
def test_attention_full_source_18bit_slots(rows_per_request, heads):
    """C = the whole source: the 2048 selected slots are token ids of the
    source (the reference feeds the LightningIndexer's ids straight in),
    several of them >= 2^14."""
    batch, source, tail = 2, 20992, 64
    total = source + tail
    bpr = math.ceil(total / 128)
    g = torch.Generator().manual_seed(7 + heads + rows_per_request)
    R = batch * rows_per_request
    scale = 1.0 / math.sqrt(576)
    t = {
        "query": torch.randn(R, heads, 512, generator=g).to(torch.bfloat16),
        "query_rope": torch.randn(R, heads, 64, generator=g).to(torch.bfloat16),
        "hbm_kv_cache": torch.randn(batch * bpr, 128, 1, 512, generator=g).to(torch.bfloat16),
        "hbm_k_rope": torch.randn(batch * bpr, 128, 1, 64, generator=g).to(torch.bfloat16),
        "hbm_block_table": torch.arange(batch * bpr, dtype=torch.int32).view(batch, bpr),
        "num_cache_tokens": torch.full((batch,), source, dtype=torch.int32),
        "actual_seq_lengths_kv": torch.full((batch,), total, dtype=torch.int32),
        "actual_seq_lengths_query": torch.arange(rows_per_request, R + 1, rows_per_request, dtype=torch.int32),
        "topk_dst_slots": torch.zeros(R, 1, TOPK, dtype=torch.int32),
    }
    for r in range(R):
        ids = torch.randperm(source, generator=g)[:TOPK]
        ids[0] = source - 1  # the largest id, past 2^14
        ids = ids.unique()
        while ids.numel() < TOPK:
            ids = torch.cat([ids, torch.randperm(source, generator=g)[:TOPK - ids.numel()]]).unique()
        t["topk_dst_slots"][r, 0] = ids[torch.randperm(TOPK, generator=g)].to(torch.int32)
    assert int(t["topk_dst_slots"].max()) >= (1 << 14)
    gold = O.sparse_tail_attention(bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]),
                                   ints(t["num_cache_tokens"]), ints(t["topk_dst_slots"]), ints(t["hbm_block_table"]),
                                   bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"]), scale, rows_per_request,
                                   dname(torch.bfloat16))
    from nanovllm_amd import dsa_offload_ops as ops

    d = {k: v.cuda() for k, v in t.items()}
    out = torch.full_like(d["query"], 7.0)
    fn = ops.sparse_tail_attention_mtp if rows_per_request > 1 else ops.sparse_tail_attention
    print(f"FULLSRC rows_per_request={rows_per_request} heads={heads}", flush=True)
    fn(d["query_rope"], d["query"], d["actual_seq_lengths_query"], d["actual_seq_lengths_kv"], d["num_cache_tokens"],
       d["topk_dst_slots"], d["hbm_block_table"], d["hbm_k_rope"], d["hbm_kv_cache"], scale, out)
    torch.cuda.synchronize()
    assert_attention_close(out, gold, label=f"full source q={rows_per_request} heads={heads}")
