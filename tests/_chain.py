"""Chain runners shared by the full-size parity tests.

``run_lim`` / ``run_copy_attend`` call the HIP library through the
reference-signature wrappers (nanovllm_amd.dsa_offload_ops, which mirror
nanovllm/models/dsa_offload_ops.py:12-248) with the views the reference
caller passes: the fused ops take ``topk_src_ids`` as [B, 2048]
(glm_mla.py:1811-1816), ``scatter_copy`` takes 3-D cache views
(glm_mla.py:1255-1258).  ``oracle_chain`` is the CPU expectation of the
copy + attention stage (HBM caches after the copy and the float64 golden)
given the LIM outputs.
"""

from __future__ import annotations

import numpy as np
import torch

from _helpers import assert_attention_close, bits, dname, ints
from oracle import dsa_oracle as O

TOPK = 2048
LIM_OUTS = ("topk_src_ids", "topk_dst_slots", "miss_counts")
MTP_OUTS = ("miss_src_ids", "miss_dst_slots")
ORACLE_KEYS = {"topk_src_ids": "src", "topk_dst_slots": "dst", "miss_counts": "miss_counts",
               "miss_src_ids": "miss_src", "miss_dst_slots": "miss_dst"}


def run_lim(t, mtp: bool) -> None:
    from nanovllm_amd import dsa_offload_ops as ops

    args = (t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
            t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"], t["cache_slots_pool"],
            t["topk_src_ids"], t["topk_dst_slots"])
    if mtp:
        ops.fused_li_manage_mtp(*args, t["miss_src_ids"], t["miss_dst_slots"], t["miss_counts"])
    else:
        ops.fused_li_manage(*args, t["miss_counts"])


def run_copy_attend(t, scale: float, mtp: bool, fused: bool) -> None:
    """offload_fuse (fused_copy_sfa(_mtp)) or offload_split (scatter_copy ->
    sparse_tail_attention(_mtp)) on the LIM outputs in ``t``."""
    from nanovllm_amd import dsa_offload_ops as ops

    B = t["num_candidate_tokens"].shape[0]
    common = (t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
              t["num_cache_tokens"], t["topk_dst_slots"])
    if fused:
        tail = (t["hbm_block_table"], t["dram_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], t["dram_k_rope"],
                t["dram_kv_cache"], scale, t["attention_out"])
        if mtp:
            ops.fused_copy_sfa_mtp(*common, t["topk_src_ids"], t["miss_src_ids"], t["miss_dst_slots"],
                                   t["miss_counts"], *tail)
        else:
            ops.fused_copy_sfa(*common, t["topk_src_ids"].view(B, TOPK), t["miss_counts"], *tail)
        return
    views = (t["hbm_k_rope"].view(-1, 128, 64), t["hbm_kv_cache"].view(-1, 128, 512),
             t["dram_k_rope"].view(-1, 128, 64), t["dram_kv_cache"].view(-1, 128, 512))
    if mtp:
        ops.scatter_copy(t["miss_src_ids"], t["miss_dst_slots"], t["miss_counts"], t["hbm_block_table"],
                         t["dram_block_table"], *views)
        ops.sparse_tail_attention_mtp(*common, t["hbm_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], scale,
                                      t["attention_out"])
    else:
        ops.scatter_copy(t["topk_src_ids"].view(B, TOPK), t["topk_dst_slots"].view(B, TOPK), t["miss_counts"],
                         t["hbm_block_table"], t["dram_block_table"], *views)
        ops.sparse_tail_attention(*common, t["hbm_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], scale,
                                  t["attention_out"])


def oracle_chain(case, lim, mtp: bool):
    """(golden attention [R,N,512] float64, HBM k_rope bits, HBM kv bits)
    after the oracle's copy + attention on ``case``'s initial HBM caches with
    the oracle LIM outputs ``lim`` (fused == split by definition,
    ut_ops/test_fused_copy_sfa.py:453-497)."""
    t = case.tensors
    dt = dname(t["query"].dtype)
    hkpe, hckv = bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"])
    common = (bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]), ints(t["num_cache_tokens"]),
              lim["dst"])
    tables = (ints(t["hbm_block_table"]), ints(t["dram_block_table"]), hkpe, hckv, bits(t["dram_k_rope"]),
              bits(t["dram_kv_cache"]), case.meta["scale"])
    if mtp:
        gold = O.fused_copy_sfa_mtp(*common, lim["miss_src"], lim["miss_dst"], lim["miss_counts"], *tables, dtype=dt)
    else:
        B = t["num_candidate_tokens"].shape[0]
        gold = O.fused_copy_sfa(*common, lim["src"].reshape(B, TOPK), lim["miss_counts"], *tables, dtype=dt)
    return gold, hkpe, hckv


def oracle_steps(case, query_names, mtp: bool):
    """The oracle through consecutive LIM -> copy -> attention steps with
    the pool and the HBM caches carried from step to step (no restore);
    step i uses the index query tensor ``query_names[i]``.  Returns one
    dict per step: the LIM outputs (``check_lim`` keys) and the pool after
    the step, the HBM cache bits after the copy, and the float64 golden."""
    t = case.tensors
    dt = dname(t["query_index"].dtype)
    B = t["num_candidate_tokens"].shape[0]
    R = t["topk_src_ids"].shape[0]
    pool = ints(t["cache_slots_pool"])
    hkpe, hckv = bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"])
    fixed = (bits(t["index_weights"]), bits(t["index_key_cache"]), ints(t["index_block_table"]),
             ints(t["num_candidate_tokens"]), ints(t["num_cache_tokens"]), ints(t["req_pool_entries"]))
    attn = (bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]), ints(t["num_cache_tokens"]))
    tables = (ints(t["hbm_block_table"]), ints(t["dram_block_table"]))
    dram = (bits(t["dram_k_rope"]), bits(t["dram_kv_cache"]))
    out = []
    for name in query_names:
        src = np.full((R, 1, TOPK), -1, np.int32)
        dst = np.full((R, 1, TOPK), -1, np.int32)
        mc = np.zeros(B, np.int32)
        if mtp:
            ms = np.full((B, 8192), -1, np.int32)
            md = np.full((B, 8192), -1, np.int32)
            O.fused_li_manage_mtp(bits(t[name]), *fixed, pool, src, dst, ms, md, mc, dtype=dt)
            lim = dict(src=src, dst=dst, miss_src=ms, miss_dst=md, miss_counts=mc)
            gold = O.fused_copy_sfa_mtp(*attn, dst, ms, md, mc, *tables, hkpe, hckv, *dram, case.meta["scale"],
                                        dtype=dt)
        else:
            O.fused_li_manage(bits(t[name]), *fixed, pool, src, dst, mc, dtype=dt)
            lim = dict(src=src, dst=dst, miss_counts=mc)
            gold = O.fused_copy_sfa(*attn, dst, src.reshape(B, TOPK), mc, *tables, hkpe, hckv, *dram,
                                    case.meta["scale"], dtype=dt)
        lim["pool"] = pool.copy()
        out.append(dict(lim=lim, hkpe=hkpe.copy(), hckv=hckv.copy(), gold=gold, query=name))
    return out


def widen_layout(t: dict, capacity: int, pad: int = 0) -> dict:
    """The model runner's table layout (nanovllm_amd.workloads.caller_layout)."""
    from nanovllm_amd.workloads import caller_layout

    return caller_layout(t, capacity, pad)


def poison_outputs(t: dict, mtp: bool) -> None:
    for k in LIM_OUTS + (MTP_OUTS if mtp else ()):
        t[k].fill_(-5)
    t["attention_out"].fill_(7.0)


def check_lim(t: dict, lim: dict, mtp: bool, label: str, pool_cols: int | None = None) -> None:
    """Every LIM output and the updated pool bit-exact (the pool's first
    ``pool_cols`` columns; the rest must be unchanged, checked by caller)."""
    counts = lim["miss_counts"]
    for k in LIM_OUTS + (MTP_OUTS if mtp else ()):
        got = ints(t[k]).reshape(lim[ORACLE_KEYS[k]].shape)
        exp = lim[ORACLE_KEYS[k]]
        if k in MTP_OUTS:  # only the first miss_counts[b] entries are defined (README_ops.md:35-51)
            valid = np.arange(exp.shape[1])[None, :] < counts[:, None]
            got, exp = np.where(valid, got, 0), np.where(valid, exp, 0)
        if not np.array_equal(got, exp):
            bad = np.argwhere(got != exp)
            raise AssertionError(f"{label}: {k} differs at {bad[:5].tolist()} ({bad.shape[0]} entries)")
    pool = ints(t["cache_slots_pool"])
    cols = pool_cols if pool_cols is not None else pool.shape[1]
    assert np.array_equal(pool[:, :cols], lim["pool"][:, :cols]), f"{label}: pool differs"


def check_copy_attend(t: dict, gold, hkpe, hckv, label: str) -> None:
    assert np.array_equal(bits(t["hbm_kv_cache"]), hckv), f"{label}: HBM kv cache differs"
    assert np.array_equal(bits(t["hbm_k_rope"]), hkpe), f"{label}: HBM k_rope cache differs"
    assert_attention_close(t["attention_out"], gold, t["attention_out"].dtype, label=label)
