"""Caller-side wrappers with the reference's signatures.

Mirror of the reference nanovllm/models/dsa_offload_ops.py:12-411: each
operator wrapper forwards to ``torch.ops.nanovllm_dsa.<op>.default`` with the
caller-owned buffers and returns ``None``; ``initialize_lidu_row(_shared)``
(the first-decode slow path, PyTorch in the reference) run on the HIP
library with the same keyword arguments, errors and return values.  Model
code written against the reference (``_lidu_update``,
``_decode_forward_mla``, the ut_ops scripts) calls these unchanged.
"""

from __future__ import annotations

import torch

from . import LIDU_MTP_QUERY_COUNT, LIDU_MTP_UNION_CAPACITY, LIDU_TOPK  # noqa: F401
from . import ops as _ops  # noqa: F401  -- registers torch.ops.nanovllm_dsa


def fused_li_manage(query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                    num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                    miss_counts) -> None:
    """Run single-query LIM into caller-owned buffers (reference dsa_offload_ops.py:12-41)."""
    torch.ops.nanovllm_dsa.fused_li_manage.default(
        query, index_weights, index_key_cache, index_block_table, num_candidate_tokens, num_cache_tokens,
        req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots, miss_counts)


def fused_li_manage_mtp(query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                        num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                        miss_src_ids, miss_dst_slots, miss_counts) -> None:
    """Run fixed-width MTP3 LIM into caller-owned buffers (reference dsa_offload_ops.py:44-77)."""
    torch.ops.nanovllm_dsa.fused_li_manage_mtp.default(
        query, index_weights, index_key_cache, index_block_table, num_candidate_tokens, num_cache_tokens,
        req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots, miss_src_ids, miss_dst_slots,
        miss_counts)


def scatter_copy(src_ids, dst_slots, copy_counts, hbm_block_table, dram_block_table, hbm_k_rope, hbm_kv_cache,
                 dram_k_rope, dram_kv_cache) -> None:
    """Copy selected CKV/KPE tokens DRAM -> HBM (reference dsa_offload_ops.py:80-101)."""
    torch.ops.nanovllm_dsa.scatter_copy.default(
        src_ids, dst_slots, copy_counts, hbm_block_table, dram_block_table, hbm_k_rope, hbm_kv_cache,
        dram_k_rope, dram_kv_cache)


def sparse_tail_attention(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                          topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache, scale_value,
                          attention_out) -> None:
    """Attend to the cached top-2048 slots plus the dense tail (reference dsa_offload_ops.py:104-131)."""
    torch.ops.nanovllm_dsa.sparse_tail_attention.default(
        query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens, topk_dst_slots,
        hbm_block_table, hbm_k_rope, hbm_kv_cache, float(scale_value), attention_out)


def sparse_tail_attention_mtp(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv,
                              num_cache_tokens, topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache,
                              scale_value, attention_out) -> None:
    """MTP3 attention, per-query causal tail (reference dsa_offload_ops.py:134-161)."""
    torch.ops.nanovllm_dsa.sparse_tail_attention_mtp.default(
        query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens, topk_dst_slots,
        hbm_block_table, hbm_k_rope, hbm_kv_cache, float(scale_value), attention_out)


def fused_copy_sfa(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                   topk_dst_slots, topk_src_ids, miss_counts, hbm_block_table, dram_block_table, hbm_k_rope,
                   hbm_kv_cache, dram_k_rope, dram_kv_cache, scale_value, attention_out) -> None:
    """Copy LIM misses and attend in one operator (reference dsa_offload_ops.py:164-199)."""
    torch.ops.nanovllm_dsa.fused_copy_sfa.default(
        query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens, topk_dst_slots,
        topk_src_ids, miss_counts, hbm_block_table, dram_block_table, hbm_k_rope, hbm_kv_cache, dram_k_rope,
        dram_kv_cache, float(scale_value), attention_out)


def fused_copy_sfa_mtp(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                       topk_dst_slots, topk_src_ids, miss_src_ids, miss_dst_slots, miss_counts, hbm_block_table,
                       dram_block_table, hbm_k_rope, hbm_kv_cache, dram_k_rope, dram_kv_cache, scale_value,
                       attention_out) -> None:
    """Copy MTP3 union misses and attend (reference dsa_offload_ops.py:202-248)."""
    torch.ops.nanovllm_dsa.fused_copy_sfa_mtp.default(
        query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens, topk_dst_slots,
        topk_src_ids, miss_src_ids, miss_dst_slots, miss_counts, hbm_block_table, dram_block_table, hbm_k_rope,
        hbm_kv_cache, dram_k_rope, dram_kv_cache, float(scale_value), attention_out)


@torch.inference_mode()
def initialize_lidu_row(*, query, weights, index_cache, index_block_table, candidate_len, cache_tokens,
                        cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table,
                        block_size):
    """First-decode top-C initialisation of one request and one layer
    (reference dsa_offload_ops.py:251-360): linear (no ReLU) index scores,
    the top ``cache_tokens`` tokens, slot i to the i-th smallest selected
    token, the pool row rewritten and the rows copied DRAM -> HBM, all on
    the GPU without a host sync.  Returns ``(hbm_kpe, hbm_ckv)``."""
    candidate_len = int(candidate_len)
    cache_tokens = int(cache_tokens)
    if cache_tokens <= 0:
        return hbm_kpe, hbm_ckv
    if cache_tokens < LIDU_TOPK:
        raise ValueError(f"LIDU nonzero cache budget must be >= {LIDU_TOPK}, got {cache_tokens}.")
    if candidate_len < cache_tokens:
        raise ValueError(f"LIDU cache budget {cache_tokens} exceeds source length {candidate_len}.")
    if candidate_len % int(block_size):
        raise ValueError("LIDU source must consist only of complete blocks.")
    _ops.lidu_init_row(query, weights, index_cache, index_block_table, candidate_len, cache_tokens, cache_slots_row,
                       hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table, int(block_size))
    return hbm_kpe, hbm_ckv


@torch.inference_mode()
def initialize_lidu_row_shared(*, cache_slots_row, cache_tokens, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv,
                               hbm_block_table, dram_block_table):
    """Copy DRAM KV to HBM for a shared IndexShare layer along the owner's
    pool row (reference dsa_offload_ops.py:363-411).  Raises RuntimeError,
    as the reference does, when the row caches a different number of tokens
    than ``cache_tokens``.  Returns ``(hbm_kpe, hbm_ckv)``."""
    cache_tokens = int(cache_tokens)
    if cache_tokens <= 0:
        return hbm_kpe, hbm_ckv
    _ops.lidu_init_row_shared(cache_slots_row, cache_tokens, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table,
                              dram_block_table)
    return hbm_kpe, hbm_ckv
