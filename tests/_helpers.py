"""Shared helpers of the parity tests (CPU side)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import dsa_oracle as O


def bits(t: torch.Tensor) -> np.ndarray:
    """16-bit float tensor -> uint16 bit patterns (numpy, on the CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def ints(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().copy()


def dname(dtype: torch.dtype) -> str:
    return "bf16" if dtype == torch.bfloat16 else "f16"


def oracle_lim(case, mtp: bool = False):
    """Run the oracle LIM on a (CPU) ChainCase; returns dict of outputs."""
    t = case.tensors
    dt = dname(t["query_index"].dtype)
    pool = ints(t["cache_slots_pool"])
    src = ints(t["topk_src_ids"])
    dst = ints(t["topk_dst_slots"])
    mc = ints(t["miss_counts"])
    args = (bits(t["query_index"]), bits(t["index_weights"]), bits(t["index_key_cache"]),
            ints(t["index_block_table"]), ints(t["num_candidate_tokens"]), ints(t["num_cache_tokens"]),
            ints(t["req_pool_entries"]), pool, src, dst)
    if mtp:
        ms = ints(t["miss_src_ids"])
        md = ints(t["miss_dst_slots"])
        O.fused_li_manage_mtp(*args, ms, md, mc, dtype=dt)
        return dict(pool=pool, src=src, dst=dst, miss_src=ms, miss_dst=md, miss_counts=mc)
    O.fused_li_manage(*args, mc, dtype=dt)
    return dict(pool=pool, src=src, dst=dst, miss_counts=mc)


def attention_errors(actual: torch.Tensor, golden: np.ndarray, dtype: torch.dtype = torch.bfloat16):
    """(max_abs, mean_rel_vs_rounded, mean_rel_vs_exact) of a 16-bit output
    against a float64 golden.  mean_rel = mean|a - g| / mean|g|."""
    a = actual.detach().float().cpu().numpy().astype(np.float64)
    g = np.asarray(golden, np.float64)
    g16 = O.bits_to_f32(O.f32_to_bits(g.astype(np.float32), dname(dtype)), dname(dtype)).astype(np.float64)
    denom = max(np.abs(g).mean(), 1e-30)
    return (float(np.abs(a - g).max()), float(np.abs(a - g16).mean() / denom), float(np.abs(a - g).mean() / denom))


# Attention tolerances (north star: max-abs 2e-2, mean-rel 1e-3 vs the fp32
# golden).  The 16-bit output rounding alone contributes ~1.35e-3 mean
# relative error against an unrounded golden (bf16: uniform error of half an
# ulp, ulp/|x| in [2^-8, 2^-7]), so mean-rel 1e-3 is checked against the
# golden rounded to the output dtype, and 3e-3 against the unrounded one.
MAX_ABS = 2e-2
MEAN_REL_ROUNDED = 1e-3
MEAN_REL_EXACT = 3e-3


def assert_attention_close(actual, golden, dtype=torch.bfloat16, label=""):
    max_abs, rel_r, rel_e = attention_errors(actual, golden, dtype)
    print(f"ATTN {label} max_abs={max_abs:.3e} mean_rel_rounded={rel_r:.3e} mean_rel_exact={rel_e:.3e}", flush=True)
    assert max_abs <= MAX_ABS, (label, max_abs)
    assert rel_r <= MEAN_REL_ROUNDED, (label, rel_r)
    assert rel_e <= MEAN_REL_EXACT, (label, rel_e)
