"""The reference's fused-copy check matrix on the GPU, against the oracle.

``fused_copy_sfa`` (README_ops.md:224-234; ut_ops/test_fused_copy_sfa.py
check mode, :531-758, graph check :806-871): 4 local attention heads,
bs in {24, 25, 48, 64}, a 20992-token source, C = 6144, a 64-token tail.
Each row attends a random 2048 of its C slots plus the tail; its first
``copy_counts`` list entries are misses with random source tokens, the
counts drawn from U[0, 2048] with row 0 at 0 and row 1 at 2048 (every list
entry a miss: 64 host tiles in one row).  As the reference checks:

* a C = 0 row beside the others (dense attention over [0, L));
* zero misses: fused and split (scatter_copy -> sparse_tail_attention);
* random misses, every miss destination poisoned first: both HBM caches
  bit-exact (copied rows from DRAM, every other row unchanged) and the
  attention within the north-star tolerance of the float64 golden, fused
  and split;
* a graph of the fused op replayed 3 times, the destinations re-poisoned
  before each replay.

MTP (README_ops.md:250-263; ut_ops/test_mtp_offload_chain.py, the entry
point of test_fused_copy_sfa_mtp.py): 2 heads, bs=4, a 20992-token source,
C = 8192, tail 64, union miss fractions 0, 1/3, 2/3 and 1 (the last request
misses its whole union): ``fused_li_manage_mtp`` then
``fused_copy_sfa_mtp`` and the split chain, eager, then the fused chain as
a graph replayed 3 times from the initial state.  Integers, pool and HBM
caches bit-exact, attention within tolerance.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _chain import check_copy_attend, check_lim, oracle_chain, poison_outputs, run_copy_attend, run_lim
from _helpers import assert_attention_close, bits, ints, oracle_lim
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

TOPK = 2048
SOURCE, CACHE, TAIL, HEADS = 20992, 6144, 64, 4


def _copy_case(batch: int, seed: int = 7, miss_min: int = 0, miss_max: int = TOPK) -> dict:
    """The inputs of ut_ops/test_fused_copy_sfa.py ``make_case`` (CPU
    tensors): private HBM blocks per row in a random order, one shared DRAM
    source read through a random permutation per row."""
    g = torch.Generator().manual_seed(seed)
    cache_blocks = math.ceil((CACHE + TAIL) / 128)
    source_blocks = SOURCE // 128
    hbm_table = torch.stack([r * cache_blocks + torch.randperm(cache_blocks, generator=g)
                             for r in range(batch)]).to(torch.int32)
    dram_table = torch.stack([torch.randperm(source_blocks, generator=g) for _ in range(batch)]).to(torch.int32)
    counts = torch.randint(miss_min, miss_max + 1, (batch,), generator=g, dtype=torch.int32)
    counts[0] = miss_min
    counts[1] = miss_max
    slots = torch.stack([torch.randperm(CACHE, generator=g)[:TOPK] for _ in range(batch)]).to(torch.int32)
    src = torch.full((batch, TOPK), -1, dtype=torch.int32)
    for r in range(batch):
        c = int(counts[r])
        src[r, :c] = torch.randperm(SOURCE, generator=g)[:c].to(torch.int32)
    bf = torch.bfloat16
    rnd = lambda *shape: torch.randn(*shape, generator=g).to(bf)  # noqa: E731
    return {
        "query": rnd(batch, HEADS, 512), "query_rope": rnd(batch, HEADS, 64),
        "topk_dst_slots": slots.view(batch, 1, TOPK).contiguous(), "topk_src_ids": src,
        "miss_counts": counts, "num_cache_tokens": torch.full((batch,), CACHE, dtype=torch.int32),
        "actual_seq_lengths_query": torch.arange(1, batch + 1, dtype=torch.int32),
        "actual_seq_lengths_kv": torch.full((batch,), CACHE + TAIL, dtype=torch.int32),
        "hbm_block_table": hbm_table, "dram_block_table": dram_table,
        "hbm_kv_cache": rnd(batch * cache_blocks, 128, 1, 512), "hbm_k_rope": rnd(batch * cache_blocks, 128, 1, 64),
        "dram_kv_cache": rnd(source_blocks, 128, 512), "dram_k_rope": rnd(source_blocks, 128, 64),
        "attention_out": torch.zeros(batch, HEADS, 512, dtype=bf),
    }


def _oracle(c: dict, scale: float):
    """(golden, HBM k_rope bits, HBM kv bits) after the copy + attention."""
    B = c["query"].shape[0]
    hkpe, hckv = bits(c["hbm_k_rope"]), bits(c["hbm_kv_cache"])
    gold = O.fused_copy_sfa(bits(c["query_rope"]), bits(c["query"]), ints(c["actual_seq_lengths_kv"]),
                            ints(c["num_cache_tokens"]), ints(c["topk_dst_slots"]),
                            ints(c["topk_src_ids"]).reshape(B, TOPK), ints(c["miss_counts"]),
                            ints(c["hbm_block_table"]), ints(c["dram_block_table"]), hkpe, hckv,
                            bits(c["dram_k_rope"]), bits(c["dram_kv_cache"]), scale)
    return gold, hkpe, hckv


def _to_device(c: dict) -> dict:
    from nanovllm_amd.host_memory import host_mapped_pair

    d = {}
    for k, v in c.items():
        if k in ("dram_kv_cache", "dram_k_rope"):
            gpu, cpu = host_mapped_pair(v.shape, v.dtype, "cuda")
            cpu.copy_(v)
            d[k] = gpu
        else:
            d[k] = v.to("cuda")
    return d


def _launch(d: dict, scale: float, fused: bool) -> None:
    from nanovllm_amd import dsa_offload_ops as ops

    B = d["query"].shape[0]
    common = (d["query_rope"], d["query"], d["actual_seq_lengths_query"], d["actual_seq_lengths_kv"],
              d["num_cache_tokens"], d["topk_dst_slots"])
    if fused:
        ops.fused_copy_sfa(*common, d["topk_src_ids"], d["miss_counts"], d["hbm_block_table"], d["dram_block_table"],
                           d["hbm_k_rope"], d["hbm_kv_cache"], d["dram_k_rope"], d["dram_kv_cache"], scale,
                           d["attention_out"])
        return
    ops.scatter_copy(d["topk_src_ids"], d["topk_dst_slots"].view(B, TOPK), d["miss_counts"], d["hbm_block_table"],
                     d["dram_block_table"], d["hbm_k_rope"].view(-1, 128, 64), d["hbm_kv_cache"].view(-1, 128, 512),
                     d["dram_k_rope"], d["dram_kv_cache"])
    ops.sparse_tail_attention(*common, d["hbm_block_table"], d["hbm_k_rope"], d["hbm_kv_cache"], scale,
                              d["attention_out"])


def _miss_rows(c: dict) -> torch.Tensor:
    """Physical HBM rows of every active miss destination."""
    rows = []
    table = c["hbm_block_table"].long()
    for r in range(c["query"].shape[0]):
        s = c["topk_dst_slots"][r, 0, :int(c["miss_counts"][r])].long()
        rows.append(table[r, s // 128] * 128 + s % 128)
    return torch.cat(rows)


def _poison(d: dict, rows: torch.Tensor, k: int = 0) -> None:
    if rows.numel():
        d["hbm_kv_cache"].view(-1, 512).index_fill_(0, rows, 37.0 + k)
        d["hbm_k_rope"].view(-1, 64).index_fill_(0, rows, -29.0 - k)


def _check(d: dict, gold, hkpe, hckv, label: str) -> None:
    assert np.array_equal(bits(d["hbm_kv_cache"]), hckv), f"{label}: HBM kv cache differs"
    assert np.array_equal(bits(d["hbm_k_rope"]), hkpe), f"{label}: HBM k_rope cache differs"
    assert torch.isfinite(d["attention_out"].float()).all(), label
    assert_attention_close(d["attention_out"], gold, torch.bfloat16, label=label)


@pytest.mark.parametrize("batch", [24, 25, 48, 64])
def test_fused_copy_sfa_reference_matrix(batch):
    scale = 1.0 / math.sqrt(576)
    base = _copy_case(batch)
    print(f"COPY MATRIX bs={batch} misses={base['miss_counts'].tolist()}", flush=True)
    assert int(base["miss_counts"][1]) == TOPK and int(base["miss_counts"][0]) == 0

    # A C = 0 row beside the others (ut_ops/test_fused_copy_sfa.py:531-560).
    c0 = {k: v.clone() for k, v in base.items()}
    c0["num_cache_tokens"][0] = 0
    c0["actual_seq_lengths_kv"][0] = TOPK + TAIL
    c0["miss_counts"][0] = 0
    gold, hkpe, hckv = _oracle(c0, scale)
    for fused in (True, False):
        d = _to_device(c0)
        _launch(d, scale, fused)
        torch.cuda.synchronize()
        _check(d, gold, hkpe, hckv, f"bs={batch} C0 row {'fused' if fused else 'split'}")
        del d

    # Zero misses (:562-597).
    z = {k: v.clone() for k, v in base.items()}
    z["miss_counts"].zero_()
    gold, hkpe, hckv = _oracle(z, scale)
    for fused in (True, False):
        d = _to_device(z)
        _launch(d, scale, fused)
        torch.cuda.synchronize()
        _check(d, gold, hkpe, hckv, f"bs={batch} zero-miss {'fused' if fused else 'split'}")
        del d

    # Random misses, destinations poisoned first (:599-758).
    rows = _miss_rows(base)
    p = {k: v.clone() for k, v in base.items()}
    p["hbm_kv_cache"].view(-1, 512)[rows] = 37.0
    p["hbm_k_rope"].view(-1, 64)[rows] = -29.0
    gold, hkpe, hckv = _oracle(p, scale)
    for fused in (True, False):
        d = _to_device(p)
        _launch(d, scale, fused)
        torch.cuda.synchronize()
        _check(d, gold, hkpe, hckv, f"bs={batch} random-miss {'fused' if fused else 'split'}")
        if fused:
            # Graph replays with the destinations re-poisoned each time (:806-871).
            dev_rows = rows.to("cuda")
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                _launch(d, scale, True)
            torch.cuda.synchronize()
            for k in range(3):
                _poison(d, dev_rows, k)
                d["attention_out"].fill_(7.0)
                torch.cuda.synchronize()
                graph.replay()
                torch.cuda.synchronize()
                _check(d, gold, hkpe, hckv, f"bs={batch} graph replay {k}")
            del graph
        del d
    torch.cuda.empty_cache()


def test_fused_copy_sfa_mtp_chain_2_heads():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(4, SOURCE, 8192, TAIL, mtp=True, attn_heads=2, miss_fracs=[0.0, 1 / 3, 2 / 3, 1.0],
                           seed=7, guard=True)
    print(f"MTP CHAIN halvings={case.meta['halvings']} miss_target={case.meta['miss_target']}", flush=True)
    lim = oracle_lim(case, mtp=True)
    gold, hkpe, hckv = oracle_chain(case, lim, mtp=True)
    counts = lim["miss_counts"]
    assert counts[0] == 0 and counts[3] > 0 and counts[3] == case.meta["miss_target"][3]
    d = case.to_device("cuda")
    t = d.tensors
    init = {k: t[k].clone() for k in ("cache_slots_pool", "hbm_kv_cache", "hbm_k_rope")}

    def restore():
        for k, v in init.items():
            t[k].copy_(v)
        poison_outputs(t, True)
        torch.cuda.synchronize()

    for fused in (True, False):
        label = f"mtp chain 2 heads {'fused' if fused else 'split'}"
        restore()
        run_lim(t, True)
        run_copy_attend(t, case.meta["scale"], True, fused)
        torch.cuda.synchronize()
        check_lim(t, lim, True, label)
        check_copy_attend(t, gold, hkpe, hckv, label)
    restore()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_lim(t, True)
        run_copy_attend(t, case.meta["scale"], True, True)
    for k in range(3):
        restore()
        graph.replay()
        torch.cuda.synchronize()
        label = f"mtp chain 2 heads graph replay {k}"
        check_lim(t, lim, True, label)
        check_copy_attend(t, gold, hkpe, hckv, label)
    del graph, d, t, init
    torch.cuda.empty_cache()
