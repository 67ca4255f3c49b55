"""oracle/torch_chain.py (the vectorised PyTorch-CPU chain timed as the CPU
baseline) against the numpy oracle, on margin-guarded workloads: top-k ids,
slots, miss counts and the pool bit-exact, the HBM caches after the copy
bit-exact, and the attention within the north-star tolerance of the float64
golden.  Covers cache budgets above 2048 (victims chosen by score), a row the
guards disable next to a C = 0 row (dense attention over [0, L)), and an
unmapped index block."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_attention_close, bits, dname, ints, oracle_lim
from oracle import dsa_oracle as O
from oracle import torch_chain as TC

TOPK = 2048


def _torch_chain(case):
    t = {k: v.clone() for k, v in case.tensors.items()}
    TC.fused_li_manage(t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
                       t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"], t["cache_slots_pool"],
                       t["topk_src_ids"], t["topk_dst_slots"], t["miss_counts"])
    B = t["query"].shape[0]
    TC.fused_copy_sfa(t["query_rope"], t["query"], t["actual_seq_lengths_kv"], t["num_cache_tokens"],
                      t["topk_dst_slots"], t["topk_src_ids"].view(B, TOPK), t["miss_counts"], t["hbm_block_table"],
                      t["dram_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], t["dram_k_rope"], t["dram_kv_cache"],
                      case.meta["scale"], t["attention_out"])
    return t


def _oracle_chain(case):
    lim = oracle_lim(case)
    t = case.tensors
    B = t["query"].shape[0]
    hkpe, hckv = bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"])
    gold = O.fused_copy_sfa(bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]),
                            ints(t["num_cache_tokens"]), lim["dst"], lim["src"].reshape(B, TOPK), lim["miss_counts"],
                            ints(t["hbm_block_table"]), ints(t["dram_block_table"]), hkpe, hckv,
                            bits(t["dram_k_rope"]), bits(t["dram_kv_cache"]), case.meta["scale"],
                            dtype=dname(t["query"].dtype))
    return lim, gold, hkpe, hckv


def _check(case, label):
    lim, gold, hkpe, hckv = _oracle_chain(case)
    got = _torch_chain(case)
    assert np.array_equal(ints(got["topk_src_ids"]), lim["src"]), label
    assert np.array_equal(ints(got["topk_dst_slots"]), lim["dst"]), label
    assert np.array_equal(ints(got["miss_counts"]), lim["miss_counts"]), label
    assert np.array_equal(ints(got["cache_slots_pool"]), lim["pool"]), label
    assert np.array_equal(bits(got["hbm_kv_cache"]), hckv), label
    assert np.array_equal(bits(got["hbm_k_rope"]), hkpe), label
    assert_attention_close(got["attention_out"], gold, got["attention_out"].dtype, label=label)
    return lim


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_torch_chain_matches_oracle(dtype):
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(4, [4096, 6144, 8192, 5120], [2048, 3072, 2560, 2048], [5, 9, 100, 1], seed=11,
                           dtype=dtype)
    lim = _check(case, f"torch chain {dtype}")
    assert int(lim["miss_counts"].sum()) > 0


def test_torch_chain_disabled_row_and_dense_row():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(3, [4096, 4096, 6144], [2048, 0, 2048], [5, 300, 17], seed=4)
    lim = _check(case, "torch chain C=0 row")
    assert lim["miss_counts"][1] == 0


def test_torch_chain_unmapped_index_block():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(2, [4096, 6144], [2048, 2048], [3, 7], seed=5)
    case.tensors["index_block_table"][1, 3] = -1  # tokens 384..511 of request 1 score -FLT_MAX
    _check(case, "torch chain unmapped block")
