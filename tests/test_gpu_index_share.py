"""IndexShare decode step on the GPU vs the oracle (BASELINE config 4's flow).

Four layers, ``full, shared, full, shared`` (reference
nanovllm/engine/dsa_offload.py:324-474): every layer has its own KV caches;
owners run LIM, members copy the owner's misses into their own HBM cache and
attend (reference glm_mla.py:1336-1406, :1542-1611).  Owner 0 starts from a
pool with misses; owner 2 starts from owner 0's post-update pool with the
same keys and query, so it selects the same tokens with no misses: a member
wired to the wrong owner copies rows it must not and fails the bit-exact
cache check.  Fused (``fused_copy_sfa(_mtp)``), split (``scatter_copy`` +
``sparse_tail_attention(_mtp)``) and group-prefetch (the split path with each
group's copies on a side stream) modes, MTP0 and MTP3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_attention_close, bits, dname, ints, oracle_lim
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

TOPK = 2048
TYPES = ("full", "shared", "full", "shared")
CACHE_NAMES = ("hbm_k_rope", "hbm_kv_cache", "dram_k_rope", "dram_kv_cache")


def _random_caches(case, seed):
    g = torch.Generator().manual_seed(seed)
    return {n: torch.randn(case[n].shape, generator=g).to(case[n].dtype) for n in CACHE_NAMES}


def _to_device(caches):
    from nanovllm_amd.host_memory import host_mapped_pair

    out = {}
    for name, v in caches.items():
        if name.startswith("dram"):
            gpu, host = host_mapped_pair(v.shape, v.dtype, torch.device("cuda"))
            host.copy_(v)
            out[name] = gpu
        else:
            out[name] = v.cuda()
    return out


def _oracle_layer(case, caches, lim, mtp):
    """Expected attention output and HBM caches of one member layer."""
    t = case.tensors
    dt = dname(t["query"].dtype)
    hkpe, hckv = bits(caches["hbm_k_rope"]), bits(caches["hbm_kv_cache"])
    common = (bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]), ints(t["num_cache_tokens"]),
              lim["dst"])
    tables = (ints(t["hbm_block_table"]), ints(t["dram_block_table"]), hkpe, hckv, bits(caches["dram_k_rope"]),
              bits(caches["dram_kv_cache"]), case.meta["scale"])
    if mtp:
        out = O.fused_copy_sfa_mtp(*common, lim["miss_src"], lim["miss_dst"], lim["miss_counts"], *tables, dtype=dt)
    else:
        B = t["query"].shape[0]
        out = O.fused_copy_sfa(*common, lim["src"].reshape(B, TOPK), lim["miss_counts"], *tables, dtype=dt)
    return out, hkpe, hckv


@pytest.mark.parametrize("mtp", [False, True])
@pytest.mark.parametrize("mode", ["fused", "split", "prefetch"])
def test_index_share_step_matches_oracle(mtp, mode):
    from nanovllm_amd.index_share import CONTEXT_FIELDS, DsaLayerCaches, IndexShareDecodeStep, IndexShareGroupManager
    from nanovllm_amd.workloads import ChainCase, make_chain_case

    print(f"INDEXSHARE mtp={mtp} mode={mode}", flush=True)
    if mtp:
        case = make_chain_case(2, [9216, 12288], [8192, 9216], [4, 33], seed=41, mtp=True)
    else:
        case = make_chain_case(2, [4096, 6144], [2048, 3072], [37, 100], seed=31)
    lim_a = oracle_lim(case, mtp=mtp)
    case_b = ChainCase(dict(case.tensors, cache_slots_pool=torch.from_numpy(lim_a["pool"].copy())), case.meta)
    lim_b = oracle_lim(case_b, mtp=mtp)
    assert int(lim_a["miss_counts"].sum()) > 0 and int(lim_b["miss_counts"].sum()) == 0
    owner_lim = {0: lim_a, 2: lim_b}
    caches = [{n: case[n] for n in CACHE_NAMES}] + [_random_caches(case, 100 + i) for i in (1, 2, 3)]
    expect = [_oracle_layer(case, caches[i], owner_lim[0 if i < 2 else 2], mtp) for i in range(4)]

    d = case.to_device("cuda")
    pool_b = torch.from_numpy(lim_a["pool"].copy()).cuda()
    layers = []
    for i in range(4):
        dc = {n: d[n] for n in CACHE_NAMES} if i == 0 else _to_device(caches[i])
        own = {}
        if i == 0:
            own = dict(index_key_cache=d["index_key_cache"], cache_slots_pool=d["cache_slots_pool"])
        elif i == 2:
            own = dict(index_key_cache=d["index_key_cache"], cache_slots_pool=pool_b)
        layers.append(DsaLayerCaches(**dc, **own))
    groups = IndexShareGroupManager(4, TYPES)
    runner = IndexShareDecodeStep(groups, layers, mtp=mtp, fused=mode == "fused", prefetch=mode == "prefetch")
    outs = [torch.full_like(d["attention_out"], 7.0) for _ in range(4)]

    def inputs(i):
        kw = dict(query_rope=d["query_rope"], query=d["query"], scale=case.meta["scale"], attention_out=outs[i])
        if groups.is_owner(i):
            kw.update(query_index=d["query_index"], index_weights=d["index_weights"])
        return kw

    runner.step({f: d[f] for f in CONTEXT_FIELDS}, inputs)
    torch.cuda.synchronize()
    B = case["query"].shape[0] // (4 if mtp else 1)
    for owner, lim in owner_lim.items():
        got = runner.owner_outputs(owner, B)
        keys = ("src", "dst", "miss_counts") + (("miss_src", "miss_dst") if mtp else ())
        names = ("topk_src_ids", "topk_dst_slots", "miss_counts") + (("miss_src_ids", "miss_dst_slots") if mtp else ())
        for k, n in zip(keys, names):
            assert np.array_equal(ints(got[n]).reshape(lim[k].shape), lim[k]), (owner, n)
        assert np.array_equal(ints(layers[owner].cache_slots_pool), lim["pool"]), owner
    for i in range(4):
        gold, hkpe, hckv = expect[i]
        assert np.array_equal(bits(layers[i].hbm_kv_cache), hckv), i
        assert np.array_equal(bits(layers[i].hbm_k_rope), hkpe), i
        assert_attention_close(outs[i], gold, label=f"layer {i} mtp={mtp} {mode}")

    # The same step captured in one HIP graph (the prefetch mode forks a copy
    # stream inside the capture): now every selection hits, and a replay must
    # give exactly what the eager step gives on the same state.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        runner.step({f: d[f] for f in CONTEXT_FIELDS}, inputs)

    def clear():
        for o in outs:
            o.fill_(7.0)
        for owner in owner_lim:
            for buf in runner.owner_outputs(owner, B).values():
                buf.fill_(-5)

    snap = []
    for run in ("replay", "eager", "replay"):
        clear()
        if run == "replay":
            graph.replay()
        else:
            runner.step({f: d[f] for f in CONTEXT_FIELDS}, inputs)
        torch.cuda.synchronize()
        snap.append([o.clone() for o in outs] + [b.clone() for owner in owner_lim
                                                 for b in runner.owner_outputs(owner, B).values()])
    assert int(runner.owner_outputs(0, B)["miss_counts"].sum()) == 0
    for a, b in zip(snap[0], snap[1]):
        assert torch.equal(a, b)
    for a, b in zip(snap[2], snap[1]):
        assert torch.equal(a, b)
