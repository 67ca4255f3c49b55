"""Prefill -> DRAM hand-over on the GPU vs the oracle, bit-exact.

* ``nvdsa_persist_prefill_blocks``: HBM blocks written into host-mapped DRAM
  caches, every DRAM byte compared (blocks not listed stay untouched, pairs
  whose ids name no block are skipped), 3-D and 4-D cache layouts.
* ``finalize_prefill_offload`` (reference glm_mla.py:850-891): the long
  request persists its full blocks and resets the owner's pool row; the short
  request maps token t to slot t and copies nothing; a shared layer leaves
  the pool row alone; Python-style block ids (negative from the end, out of
  range raises IndexError).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, ints
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _caches(hbm_blocks, dram_blocks, seed, four_d=False):
    from nanovllm_amd.host_memory import empty_host_mapped

    g = torch.Generator().manual_seed(seed)
    mid = (1,) if four_d else ()
    hckv = torch.randint(-32768, 32767, (hbm_blocks, 128, *mid, 512), generator=g, dtype=torch.int16)
    hkpe = torch.randint(-32768, 32767, (hbm_blocks, 128, *mid, 64), generator=g, dtype=torch.int16)
    dckv = empty_host_mapped((dram_blocks, 128, *mid, 512), torch.bfloat16, torch.device("cuda"))
    dkpe = empty_host_mapped((dram_blocks, 128, *mid, 64), torch.bfloat16, torch.device("cuda"))
    dckv.view(torch.int16).copy_(torch.randint(-32768, 32767, dckv.shape, generator=g, dtype=torch.int16).cuda())
    dkpe.view(torch.int16).copy_(torch.randint(-32768, 32767, dkpe.shape, generator=g, dtype=torch.int16).cuda())
    return hckv.view(torch.bfloat16).cuda(), hkpe.view(torch.bfloat16).cuda(), dckv, dkpe


@pytest.mark.parametrize("four_d", [False, True])
def test_persist_blocks_bit_exact(four_d):
    from nanovllm_amd import ops

    print(f"PERSIST four_d={four_d}", flush=True)
    hckv, hkpe, dckv, dkpe = _caches(40, 64, seed=3, four_d=four_d)
    rng = np.random.default_rng(4)
    hbm_ids = rng.permutation(40)[:30].astype(np.int32)
    dram_ids = rng.permutation(64)[:30].astype(np.int32)
    hbm_ids[5], dram_ids[9], hbm_ids[12] = -1, 64, 40  # skipped pairs
    expect_c, expect_k = bits(dckv), bits(dkpe)
    torch.cuda.synchronize()
    O.persist_blocks(bits(hckv), bits(hkpe), expect_c, expect_k, hbm_ids, dram_ids)
    ops.persist_prefill_blocks(hckv, hkpe, dckv, dkpe, torch.from_numpy(hbm_ids).cuda(),
                               torch.from_numpy(dram_ids).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(bits(dckv), expect_c)
    assert np.array_equal(bits(dkpe), expect_k)


def test_finalize_prefill_offload_long_short_shared():
    from nanovllm_amd.prefill_offload import finalize_prefill_offload

    hckv, hkpe, dckv, dkpe = _caches(24, 32, seed=5, four_d=True)
    pool = torch.full((4, 3072), 5, dtype=torch.int32, device="cuda")
    old_table = [7, 3, 21, 0, 12, 9]
    dram_table = [30, 2, 17, 5, 26, 11]
    kw = dict(old_hbm_block_table=old_table, dram_block_table=dram_table, pool_entry=2, lidu_cache_tokens=2048)
    # long request: 5 full blocks, 2 of sparse budget
    expect_c, expect_k = bits(dckv), bits(dkpe)
    torch.cuda.synchronize()
    O.persist_blocks(bits(hckv), bits(hkpe), expect_c, expect_k, old_table[:5], dram_table[:5])
    row = ints(pool[2])
    O.finalize_prefill_pool_row(row, 5, 2, 2048)
    finalize_prefill_offload(hckv, hkpe, dckv, dkpe, pool, num_full_blocks=5, num_sparse_blocks=2, **kw)
    assert np.array_equal(bits(dckv), expect_c) and np.array_equal(bits(dkpe), expect_k)
    assert np.array_equal(ints(pool[2]), row) and (ints(pool[[0, 1, 3]]) == 5).all()
    # short request: identity over 3 full blocks, nothing copied
    finalize_prefill_offload(hckv, hkpe, dckv, dkpe, pool, num_full_blocks=3, num_sparse_blocks=16, **kw)
    torch.cuda.synchronize()
    row = np.full(3072, 5, np.int32)
    O.finalize_prefill_pool_row(row, 3, 16, 2048)
    assert np.array_equal(ints(pool[2]), row)
    assert np.array_equal(bits(dckv), expect_c)
    # shared layer: pool row untouched, blocks still persisted (negative ids count from the end)
    pool[2].fill_(9)
    finalize_prefill_offload(hckv, hkpe, dckv, dkpe, pool, num_full_blocks=2, num_sparse_blocks=0,
                             is_index_share_owner=False, old_hbm_block_table=[-1, 4], dram_block_table=[0, -2],
                             pool_entry=2, lidu_cache_tokens=2048)
    O.persist_blocks(bits(hckv), bits(hkpe), expect_c, expect_k, [23, 4], [0, 30])
    assert np.array_equal(bits(dckv), expect_c) and np.array_equal(bits(dkpe), expect_k)
    assert (ints(pool[2]) == 9).all()
    with pytest.raises(IndexError):
        finalize_prefill_offload(hckv, hkpe, dckv, dkpe, pool, num_full_blocks=1, num_sparse_blocks=0,
                                 old_hbm_block_table=[24], dram_block_table=[0], pool_entry=2, lidu_cache_tokens=0)
