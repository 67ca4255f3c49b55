"""Seeded random shapes through the MTP0 and MTP3 chains vs the oracle.

The config tests fix five shapes, but the launch rules branch on the shape:
splits per row and the fused kernel's miss splits (batch, heads, miss
tiles per row), the management kernels' chunk counts (lengths, table
width), the MTP3 overlap launch (rows).  Each seed here draws a shape --
batch, per-request prompt lengths in whole 128-token blocks, cache sizes,
tails U[1,127], per-request miss fractions, 16 or 64 attention heads, the
tables' natural width or the model runner's 65536-wide layout -- and runs
LIM, then offload_fuse and offload_split, as the config tests do: LIM
outputs, the pool and both HBM caches bit-exact, attention within the
north-star tolerance.  The index query is guarded against near-ties at the
selection boundary (``make_chain_case(guard=True)``).  The edge draws add
requests that are entirely cold or entirely cached, caches up to 16383 slots,
4 to 128 heads and 64K-token prompts.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _chain import (check_copy_attend, check_lim, oracle_chain, poison_outputs, run_copy_attend, run_lim,
                    widen_layout)
from _helpers import ints, oracle_lim

pytestmark = pytest.mark.gpu

MUTABLE = ("cache_slots_pool", "hbm_kv_cache", "hbm_k_rope")
RUNNER_CAPACITY = 65536


def _mtp0_shape(seed: int):
    rng = np.random.default_rng(5000 + seed)
    batch = int(rng.integers(1, 21))
    blocks = rng.integers(24, 161, size=batch)  # 3072 .. 20480 tokens
    lens = (blocks * 128).tolist()
    caches = [int(min(L, rng.choice([2048, 3072, 4096]))) for L in lens]
    tails = rng.integers(1, 128, size=batch).tolist()
    fracs = rng.uniform(0.0, 0.5, size=batch).tolist()
    heads = int(rng.choice([16, 64]))
    wide = bool(rng.integers(0, 2))
    return batch, lens, caches, tails, fracs, heads, wide


def _mtp3_shape(seed: int):
    rng = np.random.default_rng(6000 + seed)
    batch = int(rng.integers(1, 5))
    blocks = rng.integers(64, 129, size=batch)  # 8192 .. 16384 tokens
    lens = (blocks * 128).tolist()
    # MTP3 rows need C >= min(N, 8192), and C <= 16383 (the guards' tests cover the rest)
    caches = [int(min(rng.choice([8192, L]), 16383)) for L in lens]
    tails = rng.integers(4, 128, size=batch).tolist()
    fracs = rng.uniform(0.0, 0.3, size=batch).tolist()
    heads = int(rng.choice([16, 64]))
    wide = bool(rng.integers(0, 2))
    return batch, lens, caches, tails, fracs, heads, wide


def _edge_shape(seed: int):
    """Harsher draws: whole requests cold (every selected token a miss) or fully
    cached, cache sizes up to the 16383-slot maximum, 4 to 128 attention heads,
    prompts up to 64K tokens; every third seed an MTP3 batch."""
    rng = np.random.default_rng(9000 + seed)
    mtp = seed % 3 == 2
    batch = int(rng.integers(1, 5 if mtp else 9))
    if mtp:
        blocks = rng.integers(64, 257, size=batch)
        lens = (blocks * 128).tolist()
        caches = [int(min(L, rng.choice([8192, 12288, 16383]))) for L in lens]
        tails = rng.integers(4, 128, size=batch).tolist()
    else:
        blocks = rng.integers(16, 513, size=batch)
        lens = (blocks * 128).tolist()
        caches = [int(min(L, rng.choice([2048, 4096, 8192, 12288, 16383]))) for L in lens]
        tails = rng.integers(1, 128, size=batch).tolist()
    fracs = [float(rng.choice([0.0, 0.5, 1.0])) for _ in range(batch)]
    heads = int(rng.choice([4, 16, 64, 128]))
    wide = bool(rng.integers(0, 2))
    return mtp, batch, lens, caches, tails, fracs, heads, wide


def _run(case, mtp: bool, wide: bool, tag: str) -> None:
    lim = oracle_lim(case, mtp=mtp)
    gold, hkpe, hckv = oracle_chain(case, lim, mtp)
    print(f"{tag}: oracle misses per request {ints(torch.from_numpy(lim['miss_counts'])).tolist()}", flush=True)
    d = case.to_device("cuda")
    base = d.tensors
    init = {k: base[k].clone() for k in MUTABLE}
    cap0 = base["cache_slots_pool"].shape[1]
    t = dict(base)
    if wide:
        t = widen_layout(t, RUNNER_CAPACITY, pad=0)
    wide_init = ints(t["cache_slots_pool"])
    for path in ("fused", "split"):
        label = f"{tag} S_cap={t['cache_slots_pool'].shape[1]} {path}"
        t["cache_slots_pool"].copy_(torch.from_numpy(wide_init))
        t["hbm_kv_cache"].copy_(init["hbm_kv_cache"])
        t["hbm_k_rope"].copy_(init["hbm_k_rope"])
        poison_outputs(t, mtp)
        torch.cuda.synchronize()
        print(f"RUN {label}", flush=True)
        run_lim(t, mtp)
        torch.cuda.synchronize()
        check_lim(t, lim, mtp, label, pool_cols=cap0)
        assert np.array_equal(ints(t["cache_slots_pool"])[:, cap0:], wide_init[:, cap0:]), label
        run_copy_attend(t, case.meta["scale"], mtp, fused=path == "fused")
        torch.cuda.synchronize()
        check_copy_attend(t, gold, hkpe, hckv, label)
    del d, base, init, t
    torch.cuda.empty_cache()


@pytest.mark.parametrize("seed", range(12))
def test_mtp0_chain_random_shape(seed):
    from nanovllm_amd.workloads import make_chain_case

    batch, lens, caches, tails, fracs, heads, wide = _mtp0_shape(seed)
    tag = f"mtp0 seed={seed} B={batch} heads={heads} wide={wide}"
    print(f"{tag}: lens={lens} C={caches} miss_fracs={[round(f, 2) for f in fracs]}", flush=True)
    case = make_chain_case(batch, lens, caches, tails, attn_heads=heads, miss_fracs=fracs, seed=seed, guard=True)
    _run(case, mtp=False, wide=wide, tag=tag)


@pytest.mark.parametrize("seed", range(6))
def test_mtp3_chain_random_shape(seed):
    from nanovllm_amd.workloads import make_chain_case

    batch, lens, caches, tails, fracs, heads, wide = _mtp3_shape(seed)
    tag = f"mtp3 seed={seed} B={batch} heads={heads} wide={wide}"
    print(f"{tag}: lens={lens} C={caches} miss_fracs={[round(f, 2) for f in fracs]}", flush=True)
    case = make_chain_case(batch, lens, caches, tails, attn_heads=heads, miss_fracs=fracs, seed=seed, guard=True,
                           mtp=True)
    _run(case, mtp=True, wide=wide, tag=tag)


@pytest.mark.parametrize("seed", range(12))
def test_chain_edge_shape(seed):
    from nanovllm_amd.workloads import make_chain_case

    mtp, batch, lens, caches, tails, fracs, heads, wide = _edge_shape(seed)
    tag = f"edge seed={seed} mtp={mtp} B={batch} heads={heads} wide={wide}"
    print(f"{tag}: lens={lens} C={caches} miss_fracs={fracs}", flush=True)
    case = make_chain_case(batch, lens, caches, tails, attn_heads=heads, miss_fracs=fracs, seed=seed, guard=True,
                           mtp=mtp)
    _run(case, mtp=mtp, wide=wide, tag=tag)
