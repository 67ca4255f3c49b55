"""BASELINE.json configs[4] at full size on the GPU vs the oracle: the
IndexShare decode step over 78 layers (GLM-5.2 schedule, nanovllm/config.py:26-33:
21 owners run LIM, 57 shared layers reuse their owner's selection), bs=8,
65536-token prompts, C=2048, tails U[1,127], offload_fuse and offload_split.

* Every layer has its own pinned host-mapped DRAM caches (604 MB each, 47 GB
  in all): layer i holds layer 0's rows rotated by 7*i blocks, so a member
  that copies from another layer's cache, or an owner's rows into the wrong
  layer, changes bytes.
* The owners share one guarded set of index keys and queries (each owner has
  its own copy of the key cache) but each starts from its own prior
  selection in its own pool (5-15% misses per request, drawn per owner), so
  the 21 owners' miss lists differ: a member wired to the wrong owner copies
  the wrong rows.  C == 2048 makes every victim set forced, so only the
  top-2048 boundary needs the no-near-tie guard.
* Every layer's HBM cache holds its own DRAM rows at its owner's cached slots
  (plus random tail rows), as the pool says.
* Checked after the step: each owner's top-k ids, slots, miss counts and pool
  bit-exact; each layer's HBM caches bit-exact; each layer's attention within
  the north-star tolerance.  The same state is then restored and the split
  path (scatter_copy + sparse_tail_attention per layer) must give the same.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_attention_close, bits, ints
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

L, B, N, C = 78, 8, 65536, 2048
TOPK = 2048
ROLL = 7  # blocks of rotation per layer index


def _u16(t: torch.Tensor) -> np.ndarray:
    """uint16 numpy view of a contiguous 16-bit CPU tensor (no copy)."""
    return t.view(torch.int16).numpy().view(np.uint16)


def _prior_pool(scores, table_entries, pool_shape, rng):
    """A pool whose rows cache 2048 tokens: the request's top-2048 minus a
    5-15% random subset (this step's misses) plus as many tokens from
    outside the top-2048, at a random permutation of slots [0, 2048)."""
    pool = np.full(pool_shape, -777, np.int32)
    cached_lists = []
    for b, s in enumerate(scores):
        n = s.shape[0]
        top = np.nonzero(O.topk_mask(s, TOPK))[0]
        m = int(round(rng.uniform(0.05, 0.15) * TOPK))
        misses = rng.choice(top, size=m, replace=False)
        keep = np.setdiff1d(top, misses)
        outside = np.setdiff1d(np.arange(n), top)
        fillers = rng.choice(outside, size=m, replace=False)
        cached = np.concatenate([keep, fillers])
        slots = rng.permutation(C).astype(np.int32)
        row = table_entries[b]
        pool[row] = -1
        pool[row, cached] = slots
        cached_lists.append((cached, slots))
    return pool, cached_lists


@pytest.mark.timeout(900)
def test_index_share_78_layers_full_size():
    from nanovllm_amd.host_memory import host_mapped_pair
    from nanovllm_amd.index_share import (CONTEXT_FIELDS, DsaLayerCaches, IndexShareDecodeStep,
                                          IndexShareGroupManager, glm52_indexer_types)
    from nanovllm_amd.workloads import make_chain_case

    rng = np.random.default_rng(1004)
    tails = rng.integers(1, 128, size=B)
    case = make_chain_case(B, N, C, tails, seed=4, guard=True, fast_fill=True)
    t = case.tensors
    groups = IndexShareGroupManager(L, glm52_indexer_types(L))
    owners = groups.owner_layer_idxs
    assert len(owners) == 21
    print(f"CFG4 base case built: halvings={case.meta['halvings']}", flush=True)

    # ---- oracle LIM per owner (scores once: every owner has the same keys) ----
    kc = O.bits_to_f32(bits(t["index_key_cache"]))
    q = O.bits_to_f32(bits(t["query_index"]))
    w = O.bits_to_f32(bits(t["index_weights"]))
    table = ints(t["index_block_table"])
    scores = [O.index_scores_paged(q[b], w[b], kc, table[b], N) for b in range(B)]
    del kc
    entries = ints(t["req_pool_entries"])
    pool_shape = tuple(t["cache_slots_pool"].shape)
    prior, expect_lim, cached_of = {}, {}, {}
    for j, o in enumerate(owners):
        pool, cached = _prior_pool(scores, entries, pool_shape, np.random.default_rng(5000 + j))
        prior[o] = pool.copy()
        cached_of[o] = cached
        src = np.full((B, 1, TOPK), -1, np.int32)
        dst = np.full((B, 1, TOPK), -1, np.int32)
        mc = np.zeros(B, np.int32)
        for b in range(B):
            s_, d_, m_ = O.lim_manage_row(scores[b], pool[entries[b]], N, C)
            src[b, 0], dst[b, 0], mc[b] = s_, d_, m_
        expect_lim[o] = dict(src=src, dst=dst, miss_counts=mc, pool=pool)
    print(f"CFG4 oracle LIM: misses per owner {[int(expect_lim[o]['miss_counts'].sum()) for o in owners]}",
          flush=True)

    # ---- per-layer caches: DRAM rotated per layer, HBM consistent with the owner's pool ----
    dram_ckv0, dram_kpe0 = t["dram_kv_cache"], t["dram_k_rope"]
    nb = dram_ckv0.shape[0]
    dram_table = ints(t["dram_block_table"])
    hbm_table = ints(t["hbm_block_table"])
    dev = torch.device("cuda")
    layers_host, layers = [], []
    for i in range(L):
        shift = (ROLL * i) % nb
        dram = {}
        for name, src in (("dram_kv_cache", dram_ckv0), ("dram_k_rope", dram_kpe0)):
            gpu, cpu = host_mapped_pair(src.shape, src.dtype, dev)
            cpu[: nb - shift].copy_(src[shift:])
            cpu[nb - shift:].copy_(src[:shift])
            dram[name] = (gpu, cpu)
        hckv = t["hbm_kv_cache"].clone()
        hkpe = t["hbm_k_rope"].clone()
        o = groups.owner_of(i)
        hc, hk = hckv.view(-1, 512), hkpe.view(-1, 64)
        dc, dk = dram["dram_kv_cache"][1].view(-1, 512), dram["dram_k_rope"][1].view(-1, 64)
        for b, (cached, slots) in enumerate(cached_of[o]):
            srow = torch.from_numpy(dram_table[b, cached // 128].astype(np.int64) * 128 + cached % 128)
            drow = torch.from_numpy(hbm_table[b, slots // 128].astype(np.int64) * 128 + slots % 128)
            hc[drow] = dc[srow]
            hk[drow] = dk[srow]
        layers_host.append(dict(hbm_kv_cache=hckv, hbm_k_rope=hkpe, dram_kv_cache=dram["dram_kv_cache"][1],
                                dram_k_rope=dram["dram_k_rope"][1]))
        layers.append(dict(hbm_kv_cache=hckv.to(dev), hbm_k_rope=hkpe.to(dev), dram_kv_cache=dram["dram_kv_cache"][0],
                           dram_k_rope=dram["dram_k_rope"][0]))
    print("CFG4 layer caches built", flush=True)

    # ---- oracle copy + attention per layer ----
    common = (bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]), ints(t["num_cache_tokens"]))
    expect_layers = []
    for i in range(L):
        lim = expect_lim[groups.owner_of(i)]
        hk, hc = bits(layers_host[i]["hbm_k_rope"]), bits(layers_host[i]["hbm_kv_cache"])
        gold = O.fused_copy_sfa(*common, lim["dst"], lim["src"].reshape(B, TOPK), lim["miss_counts"], hbm_table,
                                dram_table, hk, hc, _u16(layers_host[i]["dram_k_rope"]),
                                _u16(layers_host[i]["dram_kv_cache"]), case.meta["scale"])
        expect_layers.append((gold, hk, hc))
    print("CFG4 oracle copy + attention done", flush=True)

    # ---- the GPU step ----
    d = {k: v.to(dev) for k, v in t.items() if k not in ("dram_kv_cache", "dram_k_rope", "hbm_kv_cache",
                                                          "hbm_k_rope", "cache_slots_pool")}
    pools = {o: torch.from_numpy(prior[o]).to(dev) for o in owners}
    keys = {o: d["index_key_cache"] if o == 0 else d["index_key_cache"].clone() for o in owners}
    stack = []
    for i in range(L):
        own = dict(index_key_cache=keys[i], cache_slots_pool=pools[i]) if groups.is_owner(i) else {}
        stack.append(DsaLayerCaches(hbm_k_rope=layers[i]["hbm_k_rope"], hbm_kv_cache=layers[i]["hbm_kv_cache"],
                                    dram_k_rope=layers[i]["dram_k_rope"], dram_kv_cache=layers[i]["dram_kv_cache"],
                                    **own))
    init_hbm = [(lay["hbm_kv_cache"].clone(), lay["hbm_k_rope"].clone()) for lay in layers]
    outs = [torch.full_like(d["attention_out"], 7.0) for _ in range(L)]
    ctx = {f: d[f] for f in CONTEXT_FIELDS}

    def inputs(i):
        kw = dict(query_rope=d["query_rope"], query=d["query"], scale=case.meta["scale"], attention_out=outs[i])
        if groups.is_owner(i):
            kw.update(query_index=d["query_index"], index_weights=d["index_weights"])
        return kw

    for mode in ("fused", "split"):
        for o in owners:
            pools[o].copy_(torch.from_numpy(prior[o]))
        for i in range(L):
            layers[i]["hbm_kv_cache"].copy_(init_hbm[i][0])
            layers[i]["hbm_k_rope"].copy_(init_hbm[i][1])
            outs[i].fill_(7.0)
        runner = IndexShareDecodeStep(groups, stack, fused=mode == "fused")
        torch.cuda.synchronize()
        print(f"CFG4 RUN {mode}: 78-layer step", flush=True)
        runner.step(ctx, inputs)
        torch.cuda.synchronize()
        for o in owners:
            got = runner.owner_outputs(o, B)
            exp = expect_lim[o]
            assert np.array_equal(ints(got["topk_src_ids"]), exp["src"]), (mode, o, "src")
            assert np.array_equal(ints(got["topk_dst_slots"]), exp["dst"]), (mode, o, "dst")
            assert np.array_equal(ints(got["miss_counts"]), exp["miss_counts"]), (mode, o, "miss_counts")
            assert np.array_equal(ints(pools[o]), exp["pool"]), (mode, o, "pool")
        for i in range(L):
            gold, hk, hc = expect_layers[i]
            assert np.array_equal(bits(layers[i]["hbm_kv_cache"]), hc), (mode, i, "hbm_kv_cache")
            assert np.array_equal(bits(layers[i]["hbm_k_rope"]), hk), (mode, i, "hbm_k_rope")
            assert_attention_close(outs[i], gold, label=f"cfg4 {mode} layer {i}")
        print(f"CFG4 {mode}: 21 owners and 78 layers match", flush=True)
