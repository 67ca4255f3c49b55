"""DsaLayerGraph (the decode graph runner, reference
nanovllm/engine/full_decode_graph.py:546-720) on the GPU vs the oracle.

* A step captured at a larger batch and replayed with the runtime batch
  (padded rows) must give the oracle's integer outputs, pool and HBM caches
  bit for bit and the oracle's attention within tolerance, on every replay
  (the persistent state is restored between replays, with eager work and
  synchronisations in between), leave the padded rows inert (no misses,
  zero output) and leave the state untouched by its capture warm-up.
  MTP0 and MTP3.
* More than 32 graphs captured in ascending batch order (the reference
  captures its sizes in order, full_decode_graph.py:525-585; PyTorch hands
  out 32 pool streams round-robin) each keep their own workspace: after all
  captures the first graph, the largest one at a small runtime batch and a
  second one at a runtime batch smaller than an earlier replay all match the
  oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _chain import oracle_chain
from _helpers import assert_attention_close, bits, ints, oracle_lim

pytestmark = pytest.mark.gpu

STATE = ("cache_slots_pool", "hbm_kv_cache", "hbm_k_rope")
RUNTIME = ("query_index", "index_weights", "index_block_table", "num_candidate_tokens", "num_cache_tokens",
           "req_pool_entries", "query_rope", "query", "actual_seq_lengths_query", "actual_seq_lengths_kv",
           "hbm_block_table", "dram_block_table")
PER_REQUEST = ("index_block_table", "num_candidate_tokens", "num_cache_tokens", "req_pool_entries",
               "actual_seq_lengths_query", "actual_seq_lengths_kv", "hbm_block_table", "dram_block_table",
               "miss_counts", "miss_src_ids", "miss_dst_slots")
PER_ROW = ("query_index", "index_weights", "query_rope", "query", "topk_src_ids", "topk_dst_slots",
           "attention_out")


def _first_requests(case, n: int):
    """The step restricted to its first n requests (same persistent state)."""
    from nanovllm_amd.workloads import ChainCase

    q = case.meta["queries"]
    t = dict(case.tensors)
    for k in PER_REQUEST:
        if k in t:
            t[k] = t[k][:n].clone()
    for k in PER_ROW:
        t[k] = t[k][:n * q].clone()
    meta = dict(case.meta, batch=n)
    return ChainCase(t, meta)


def _expect(case, mtp: bool):
    lim = oracle_lim(case, mtp=mtp)
    gold, hkpe, hckv = oracle_chain(case, lim, mtp)
    return lim, gold, hkpe, hckv


def _check(out, state, exp, mtp, label):
    lim, gold, hkpe, hckv = exp
    names = {"topk_src_ids": "src", "topk_dst_slots": "dst", "miss_counts": "miss_counts"}
    if mtp:
        names.update(miss_src_ids="miss_src", miss_dst_slots="miss_dst")
    for k, ok in names.items():
        assert np.array_equal(ints(out[k]).reshape(lim[ok].shape), lim[ok]), (label, k)
    assert np.array_equal(ints(state["cache_slots_pool"]), lim["pool"]), (label, "pool")
    assert np.array_equal(bits(state["hbm_kv_cache"]), hckv), (label, "hbm_kv_cache")
    assert np.array_equal(bits(state["hbm_k_rope"]), hkpe), (label, "hbm_k_rope")
    assert_attention_close(out["attention_out"], gold, label=label)


def _graph(batch, t, scale, mtp):
    from nanovllm_amd.decode_graph import DsaLayerGraph

    return DsaLayerGraph(batch, index_key_cache=t["index_key_cache"], cache_slots_pool=t["cache_slots_pool"],
                         hbm_k_rope=t["hbm_k_rope"], hbm_kv_cache=t["hbm_kv_cache"], dram_k_rope=t["dram_k_rope"],
                         dram_kv_cache=t["dram_kv_cache"], hbm_block_columns=t["hbm_block_table"].shape[1] + 3,
                         dram_block_columns=t["dram_block_table"].shape[1] + 1, heads=t["query"].shape[1],
                         index_heads=t["query_index"].shape[1], scale=scale, mtp=mtp)


@pytest.mark.parametrize("mtp", [False, True])
def test_padded_graph_replays_match_oracle(mtp):
    from nanovllm_amd.workloads import make_chain_case

    if mtp:
        case = make_chain_case(2, [9216, 12288], [8192, 9216], [4, 33], seed=31, mtp=True)
    else:
        case = make_chain_case(3, [8192, 12288, 16384], [2048, 4096, 2048], [5, 60, 127], seed=31)
    print(f"DECODE GRAPH mtp={mtp}", flush=True)
    exp = _expect(case, mtp)
    assert int(exp[0]["miss_counts"].sum()) > 0, "the step must copy rows"
    d = case.to_device("cuda")
    t = d.tensors
    B = t["num_candidate_tokens"].shape[0]
    init = {k: t[k].clone() for k in STATE}
    g = _graph(B + 2, t, case.meta["scale"], mtp)
    g.capture()
    torch.cuda.synchronize()
    for k in STATE:  # the capture warm-up ran padded rows only
        assert torch.equal(t[k], init[k]), k
    runtime = {k: t[k] for k in RUNTIME}
    q = 4 if mtp else 1
    for rep in range(3):
        for k in STATE:
            t[k].copy_(init[k])
        torch.cuda.synchronize()
        out = g.replay(**runtime)
        torch.cuda.synchronize()
        _check(out, t, exp, mtp, f"replay {rep} mtp={mtp}")
        assert (ints(g.outputs["miss_counts"][B:]) == 0).all()
        assert (bits(g.outputs["attention_out"][B * q:]) == 0).all()
    assert g.replay_count == 3
    with pytest.raises(ValueError, match="exceeds"):
        big = dict(runtime)
        big["num_candidate_tokens"] = torch.zeros(B + 3, dtype=torch.int32, device="cuda")
        g.copy_runtime_inputs(**big)


def test_many_captured_graphs_keep_their_workspaces():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(3, [8192, 12288, 16384], [2048, 4096, 2048], [5, 60, 127], seed=33)
    exp3 = _expect(case, False)
    exp2 = _expect(_first_requests(case, 2), False)
    assert int(exp2[0]["miss_counts"].sum()) > 0
    d = case.to_device("cuda")
    t = d.tensors
    init = {k: t[k].clone() for k in STATE}
    sizes = list(range(3, 3 + 34))  # 34 graphs, ascending batch: every capture grows the operators' scratch needs
    graphs = []
    for size in sizes:
        g = _graph(size, t, case.meta["scale"], False)
        g.capture()
        graphs.append(g)
    torch.cuda.synchronize()
    print(f"captured {len(graphs)} graphs, batch {sizes[0]}..{sizes[-1]}", flush=True)
    full = {k: t[k] for k in RUNTIME}
    two = {k: v[:2] for k, v in full.items()}  # MTP0: one row per request
    for label, g, runtime, exp in (("first graph, batch 3", graphs[0], full, exp3),
                                   ("largest graph, batch 3", graphs[-1], full, exp3),
                                   ("second graph, batch 2", graphs[1], two, exp2),
                                   ("first graph again, batch 3", graphs[0], full, exp3)):
        for k in STATE:
            t[k].copy_(init[k])
        torch.cuda.synchronize()
        print(f"REPLAY {label}", flush=True)
        out = g.replay(**runtime)
        torch.cuda.synchronize()
        _check(out, t, exp, False, label)
