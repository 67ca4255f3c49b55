"""Prefill -> DRAM hand-over of one attention layer on MI355X.

Mirrors ``GlmMLAAttention.finalize_prefill_offload`` (reference
nanovllm/models/glm_mla.py:850-889) as a function of the layer's caches and
the request's fields (the engine passes ``seq`` and reads
``num_prefill_full_blocks``, ``num_sparse_blocks``, ``offload_pool_entry``,
``lidu_cache_tokens`` and ``dram_block_table`` from it):

* the IndexShare owner resets its pool row to -1 (:857-865);
* a short request (every full block fits the sparse budget) keeps its KV in
  HBM and the owner maps source token t to slot t (:866-880);
* otherwise every full prefill block is persisted HBM -> DRAM, CKV and KPE,
  in ONE launch (``nvdsa_persist_prefill_blocks``) instead of a synchronous
  ``.copy_`` per cache and block (:882-889), then the device is synchronised
  as in the reference (:890-891), because the engine releases the HBM blocks
  right after this call (nanovllm/engine/dsa_offload.py:228-246).

Block ids follow Python indexing: a negative id counts from the end and an
id out of range raises ``IndexError``, as ``cache[block]`` does.
"""

from __future__ import annotations

import torch

from . import ops


def _block_ids(ids, n_blocks: int, name: str) -> list[int]:
    out = []
    for b in ids:
        b = int(b)
        if b < -n_blocks or b >= n_blocks:
            raise IndexError(f"index {b} is out of bounds for dimension 0 with size {n_blocks} ({name})")
        out.append(b + n_blocks if b < 0 else b)
    return out


def persist_prefill_blocks(ckv_cache, kpe_cache, dram_ckv_cache, dram_kpe_cache, hbm_blocks, dram_blocks) -> None:
    """dram_*[dram_blocks[i]] = *_cache[hbm_blocks[i]] for every i, one launch
    on the current stream (no host sync)."""
    if len(hbm_blocks) != len(dram_blocks):
        raise ValueError("hbm_blocks and dram_blocks must have the same length")
    if not hbm_blocks:
        return
    h = _block_ids(hbm_blocks, ckv_cache.shape[0], "hbm")
    d = _block_ids(dram_blocks, dram_ckv_cache.shape[0], "dram")
    dev = ckv_cache.device
    ids = torch.tensor([h, d], dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
    ops.persist_prefill_blocks(ckv_cache, kpe_cache, dram_ckv_cache, dram_kpe_cache, ids[0], ids[1])


def finalize_prefill_offload(ckv_cache, kpe_cache, dram_ckv_cache, dram_kpe_cache, lidu_cache_slots, *,
                             old_hbm_block_table, dram_block_table, num_full_blocks: int, num_sparse_blocks: int,
                             pool_entry: int, lidu_cache_tokens: int, is_index_share_owner: bool = True,
                             block_size: int = 128) -> None:
    """One layer's prefill hand-over (reference glm_mla.py:850-891)."""
    num_full_blocks = int(num_full_blocks)
    if is_index_share_owner:
        lidu_cache_slots[int(pool_entry)].fill_(-1)
    if int(num_sparse_blocks) >= num_full_blocks:
        if is_index_share_owner and int(lidu_cache_tokens) > 0 and num_full_blocks > 0:
            source_tokens = num_full_blocks * int(block_size)
            lidu_cache_slots[int(pool_entry), :source_tokens].copy_(
                torch.arange(source_tokens, dtype=torch.int32, device=lidu_cache_slots.device))
        return
    persist_prefill_blocks(ckv_cache, kpe_cache, dram_ckv_cache, dram_kpe_cache,
                           list(old_hbm_block_table[:num_full_blocks]), list(dram_block_table[:num_full_blocks]))
    torch.cuda.synchronize(ckv_cache.device)


__all__ = ["finalize_prefill_offload", "persist_prefill_blocks"]
