"""``torch.ops.nanovllm_dsa`` on PyTorch-ROCm, backed by libnvdsa.so.

Importing this module registers the seven DSA offload operators and the
indexer's query RoPE under the reference's namespace and schemas (reference
csrc/nanovllm_ascend_ops/bindings/nanovllm_ops.cpp:645-696 and :713-714,
registered on import by nanovllm/ops/__init__.py:38-50):

* a CUDA-key implementation that hands plain tensor descriptors to the C ABI
  and launches on the current HIP stream (the counterpart of the PrivateUse1
  implementations, nanovllm_ops.cpp:731-738);
* a Meta implementation that does nothing, so the operators are traceable
  and graph-capturable like the reference's (nanovllm_ops.cpp:750-757).

Every operator returns ``None`` and writes caller-owned buffers in place.
There is no CPU implementation and no fallback path: a call whose tensors
are not on the GPU fails in the dispatcher, and a call the C ABI rejects
raises ``RuntimeError`` with the ABI's message (the reference's TORCH_CHECK
behaviour).

DRAM caches (``dram_k_rope`` / ``dram_kv_cache``) may be GPU-typed tensors
over host-mapped memory (:func:`nanovllm_amd.host_memory.empty_host_mapped`)
or pinned CPU tensors; the GPU reads them over the host link.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

NAMESPACE = "nanovllm_dsa"

# Exact schema strings of the reference (nanovllm_ops.cpp:646-696).
SCHEMAS = {
    "fused_li_manage": (
        "fused_li_manage(Tensor query, Tensor index_weights,"
        " Tensor index_key_cache, Tensor index_block_table,"
        " Tensor num_candidate_tokens, Tensor num_cache_tokens,"
        " Tensor req_pool_entries, Tensor(a!) cache_slots_pool,"
        " Tensor(b!) topk_src_ids, Tensor(c!) topk_dst_slots,"
        " Tensor(d!) miss_counts) -> ()"
    ),
    "fused_li_manage_mtp": (
        "fused_li_manage_mtp(Tensor query, Tensor index_weights,"
        " Tensor index_key_cache, Tensor index_block_table,"
        " Tensor num_candidate_tokens, Tensor num_cache_tokens,"
        " Tensor req_pool_entries, Tensor(a!) cache_slots_pool,"
        " Tensor(b!) topk_src_ids, Tensor(c!) topk_dst_slots,"
        " Tensor(d!) miss_src_ids, Tensor(e!) miss_dst_slots,"
        " Tensor(f!) miss_counts) -> ()"
    ),
    "scatter_copy": (
        "scatter_copy(Tensor src_ids, Tensor dst_slots, Tensor copy_counts,"
        " Tensor hbm_block_table, Tensor dram_block_table,"
        " Tensor(a!) hbm_k_rope, Tensor(b!) hbm_kv_cache,"
        " Tensor dram_k_rope, Tensor dram_kv_cache) -> ()"
    ),
    "sparse_tail_attention": (
        "sparse_tail_attention(Tensor query_rope, Tensor query,"
        " Tensor actual_seq_lengths_query, Tensor actual_seq_lengths_kv,"
        " Tensor num_cache_tokens, Tensor topk_dst_slots,"
        " Tensor hbm_block_table, Tensor hbm_k_rope, Tensor hbm_kv_cache,"
        " float scale_value, Tensor(a!) attention_out) -> ()"
    ),
    "sparse_tail_attention_mtp": (
        "sparse_tail_attention_mtp(Tensor query_rope, Tensor query,"
        " Tensor actual_seq_lengths_query, Tensor actual_seq_lengths_kv,"
        " Tensor num_cache_tokens, Tensor topk_dst_slots,"
        " Tensor hbm_block_table, Tensor hbm_k_rope, Tensor hbm_kv_cache,"
        " float scale_value, Tensor(a!) attention_out) -> ()"
    ),
    "fused_copy_sfa": (
        "fused_copy_sfa(Tensor query_rope, Tensor query,"
        " Tensor actual_seq_lengths_query, Tensor actual_seq_lengths_kv,"
        " Tensor num_cache_tokens, Tensor topk_dst_slots,"
        " Tensor topk_src_ids, Tensor miss_counts,"
        " Tensor hbm_block_table, Tensor dram_block_table,"
        " Tensor(a!) hbm_k_rope, Tensor(b!) hbm_kv_cache,"
        " Tensor dram_k_rope, Tensor dram_kv_cache, float scale_value,"
        " Tensor(c!) attention_out) -> ()"
    ),
    "fused_copy_sfa_mtp": (
        "fused_copy_sfa_mtp(Tensor query_rope, Tensor query,"
        " Tensor actual_seq_lengths_query, Tensor actual_seq_lengths_kv,"
        " Tensor num_cache_tokens, Tensor topk_dst_slots,"
        " Tensor topk_src_ids, Tensor miss_src_ids, Tensor miss_dst_slots,"
        " Tensor miss_counts, Tensor hbm_block_table,"
        " Tensor dram_block_table, Tensor(a!) hbm_k_rope,"
        " Tensor(b!) hbm_kv_cache, Tensor dram_k_rope,"
        " Tensor dram_kv_cache, float scale_value,"
        " Tensor(c!) attention_out) -> ()"
    ),
    # nanovllm_ops.cpp:713-714
    "dsa_indexer_query_rope_inplace": (
        "dsa_indexer_query_rope_inplace(Tensor(a!) q_inout, Tensor cos,"
        " Tensor sin, int rope_dim) -> ()"
    ),
}

_D = _lib.describe
_L = _lib.lib


def _ref(d: _lib.NvdsaTensor):
    return ctypes.byref(d)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch memory for one operator call, from torch's caching allocator.

    The block is allocated on the current stream and released when the call
    returns; the allocator reuses it only for work ordered after this call
    on that stream, so the kernels may still be running when it is freed.
    Under HIP-graph capture the block comes from the graph's private pool
    and stays reserved for as long as the graph lives, so every captured
    graph replays against its own workspace, whatever is captured or run
    after it.  In steady state no call reaches hipMalloc."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _fused_li_manage(query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                     num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                     miss_counts) -> None:
    descs = [_D(t) for t in (query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                             num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                             miss_counts)]
    nbytes = _L.nvdsa_fused_li_manage_workspace_size(query.shape[0] if query.dim() else 0,
                                                     index_block_table.shape[-1] * 128 if index_block_table.dim() == 2 else 0,
                                                     query.shape[1] if query.dim() > 1 else 0)
    ws = _workspace(query.device, nbytes)
    _lib.check(_L.nvdsa_fused_li_manage(*map(_ref, descs), ws.data_ptr(), ws.numel(), _stream_of(query)))


def _fused_li_manage_mtp(query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                         num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                         miss_src_ids, miss_dst_slots, miss_counts) -> None:
    descs = [_D(t) for t in (query, index_weights, index_key_cache, index_block_table, num_candidate_tokens,
                             num_cache_tokens, req_pool_entries, cache_slots_pool, topk_src_ids, topk_dst_slots,
                             miss_src_ids, miss_dst_slots, miss_counts)]
    batch = req_pool_entries.shape[0] if req_pool_entries.dim() == 1 else 0
    nbytes = _L.nvdsa_fused_li_manage_mtp_workspace_size(
        batch, index_block_table.shape[-1] * 128 if index_block_table.dim() == 2 else 0,
        query.shape[1] if query.dim() > 1 else 0)
    ws = _workspace(query.device, nbytes)
    _lib.check(_L.nvdsa_fused_li_manage_mtp(*map(_ref, descs), ws.data_ptr(), ws.numel(), _stream_of(query)))


def _scatter_copy(src_ids, dst_slots, copy_counts, hbm_block_table, dram_block_table, hbm_k_rope, hbm_kv_cache,
                  dram_k_rope, dram_kv_cache) -> None:
    descs = [_D(t) for t in (src_ids, dst_slots, copy_counts, hbm_block_table, dram_block_table, hbm_k_rope,
                             hbm_kv_cache, dram_k_rope, dram_kv_cache)]
    _lib.check(_L.nvdsa_scatter_copy(*map(_ref, descs), _stream_of(hbm_kv_cache)))


def _attention_workspace(query: torch.Tensor) -> torch.Tensor:
    rows = query.shape[0] if query.dim() == 3 else 0
    heads = query.shape[1] if query.dim() == 3 else 0
    nbytes = _L.nvdsa_sparse_tail_attention_workspace_size(rows, heads, 0)
    return _workspace(query.device, nbytes)


def _sparse_tail_attention(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                           topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache, scale_value,
                           attention_out) -> None:
    descs = [_D(t) for t in (query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                             topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache)]
    out = _D(attention_out)
    ws = _attention_workspace(query)
    _lib.check(_L.nvdsa_sparse_tail_attention(*map(_ref, descs), float(scale_value), _ref(out), ws.data_ptr(),
                                              ws.numel(), _stream_of(query)))


def _sparse_tail_attention_mtp(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv,
                               num_cache_tokens, topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache,
                               scale_value, attention_out) -> None:
    descs = [_D(t) for t in (query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                             topk_dst_slots, hbm_block_table, hbm_k_rope, hbm_kv_cache)]
    out = _D(attention_out)
    ws = _attention_workspace(query)
    _lib.check(_L.nvdsa_sparse_tail_attention_mtp(*map(_ref, descs), float(scale_value), _ref(out), ws.data_ptr(),
                                                  ws.numel(), _stream_of(query)))


def _fused_copy_sfa(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                    topk_dst_slots, topk_src_ids, miss_counts, hbm_block_table, dram_block_table, hbm_k_rope,
                    hbm_kv_cache, dram_k_rope, dram_kv_cache, scale_value, attention_out) -> None:
    descs = [_D(t) for t in (query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                             topk_dst_slots, topk_src_ids, miss_counts, hbm_block_table, dram_block_table,
                             hbm_k_rope, hbm_kv_cache, dram_k_rope, dram_kv_cache)]
    out = _D(attention_out)
    ws = _attention_workspace(query)
    _lib.check(_L.nvdsa_fused_copy_sfa(*map(_ref, descs), float(scale_value), _ref(out), ws.data_ptr(),
                                       ws.numel(), _stream_of(query)))


def _fused_copy_sfa_mtp(query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                        topk_dst_slots, topk_src_ids, miss_src_ids, miss_dst_slots, miss_counts, hbm_block_table,
                        dram_block_table, hbm_k_rope, hbm_kv_cache, dram_k_rope, dram_kv_cache, scale_value,
                        attention_out) -> None:
    descs = [_D(t) for t in (query_rope, query, actual_seq_lengths_query, actual_seq_lengths_kv, num_cache_tokens,
                             topk_dst_slots, topk_src_ids, miss_src_ids, miss_dst_slots, miss_counts,
                             hbm_block_table, dram_block_table, hbm_k_rope, hbm_kv_cache, dram_k_rope,
                             dram_kv_cache)]
    out = _D(attention_out)
    ws = _attention_workspace(query)
    _lib.check(_L.nvdsa_fused_copy_sfa_mtp(*map(_ref, descs), float(scale_value), _ref(out), ws.data_ptr(),
                                           ws.numel(), _stream_of(query)))


def lidu_init_row(query, weights, index_cache, index_block_table, candidate_len, cache_tokens, cache_slots_row,
                  hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table, block_size) -> None:
    """nvdsa_initialize_lidu_row on the current stream (no host sync)."""
    descs = [_D(t) for t in (query, weights, index_cache, index_block_table)]
    rest = [_D(t) for t in (cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table,
                            dram_block_table)]
    nbytes = _L.nvdsa_initialize_lidu_row_workspace_size(cache_slots_row.shape[0] if cache_slots_row.dim() else 0)
    ws = _workspace(query.device, nbytes)
    _lib.check(_L.nvdsa_initialize_lidu_row(*map(_ref, descs), int(candidate_len), int(cache_tokens),
                                            *map(_ref, rest), int(block_size), ws.data_ptr(), ws.numel(),
                                            _stream_of(query)))


def lidu_init_row_shared(cache_slots_row, cache_tokens, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table,
                         dram_block_table) -> None:
    """nvdsa_initialize_lidu_row_shared (synchronises the current stream once)."""
    descs = [_D(t) for t in (hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table)]
    nbytes = _L.nvdsa_initialize_lidu_row_workspace_size(cache_slots_row.shape[0] if cache_slots_row.dim() else 0)
    ws = _workspace(hbm_kpe.device, nbytes)
    _lib.check(_L.nvdsa_initialize_lidu_row_shared(_ref(_D(cache_slots_row)), int(cache_tokens), *map(_ref, descs),
                                                   ws.data_ptr(), ws.numel(), _stream_of(hbm_kpe)))


def _dsa_indexer_query_rope_inplace(q_inout, cos, sin, rope_dim) -> None:
    descs = [_D(t) for t in (q_inout, cos, sin)]
    _lib.check(_L.nvdsa_dsa_indexer_query_rope_inplace(*map(_ref, descs), int(rope_dim), _stream_of(q_inout)))


def indexer_project_query_only(hidden_states, q_c, cos, sin, wq_b_weight, weights_proj_weight, q_index_out,
                               index_weights_out, n_head, head_dim, rope_dim, score_scale) -> None:
    """nvdsa_dsa_indexer_project_query_only on the current stream.  Pass
    ``weights_proj_weight`` and ``index_weights_out`` as None to project q
    only."""
    descs = [_D(t) for t in (hidden_states, q_c, cos, sin, wq_b_weight)]
    wp = _D(weights_proj_weight) if weights_proj_weight is not None else None
    qo = _D(q_index_out)
    wo = _D(index_weights_out) if index_weights_out is not None else None
    _lib.check(_L.nvdsa_dsa_indexer_project_query_only(
        *map(_ref, descs), _ref(wp) if wp is not None else None, _ref(qo), _ref(wo) if wo is not None else None,
        int(n_head), int(head_dim), int(rope_dim), float(score_scale), _stream_of(q_c)))


def persist_prefill_blocks(hbm_kv_cache, hbm_k_rope, dram_kv_cache, dram_k_rope, hbm_block_ids,
                           dram_block_ids) -> None:
    """nvdsa_persist_prefill_blocks on the current stream (no host sync)."""
    descs = [_D(t) for t in (hbm_kv_cache, hbm_k_rope, dram_kv_cache, dram_k_rope, hbm_block_ids, dram_block_ids)]
    _lib.check(_L.nvdsa_persist_prefill_blocks(*map(_ref, descs), _stream_of(hbm_kv_cache)))


IMPLS = {
    "fused_li_manage": _fused_li_manage,
    "fused_li_manage_mtp": _fused_li_manage_mtp,
    "scatter_copy": _scatter_copy,
    "sparse_tail_attention": _sparse_tail_attention,
    "sparse_tail_attention_mtp": _sparse_tail_attention_mtp,
    "fused_copy_sfa": _fused_copy_sfa,
    "fused_copy_sfa_mtp": _fused_copy_sfa_mtp,
    "dsa_indexer_query_rope_inplace": _dsa_indexer_query_rope_inplace,
}


def _meta(*args, **kwargs) -> None:
    return None


def _register() -> torch.library.Library | None:
    if hasattr(torch.ops, NAMESPACE) and hasattr(getattr(torch.ops, NAMESPACE), "scatter_copy"):
        try:
            getattr(torch.ops, NAMESPACE).scatter_copy.default
            return None  # already registered in this process
        except (AttributeError, RuntimeError):
            pass
    library = torch.library.Library(NAMESPACE, "DEF")
    for name, schema in SCHEMAS.items():
        library.define(schema)
        library.impl(name, IMPLS[name], "CUDA")
        library.impl(name, _meta, "Meta")
    return library


_LIBRARY = _register()

fused_li_manage = torch.ops.nanovllm_dsa.fused_li_manage.default
fused_li_manage_mtp = torch.ops.nanovllm_dsa.fused_li_manage_mtp.default
scatter_copy = torch.ops.nanovllm_dsa.scatter_copy.default
sparse_tail_attention = torch.ops.nanovllm_dsa.sparse_tail_attention.default
sparse_tail_attention_mtp = torch.ops.nanovllm_dsa.sparse_tail_attention_mtp.default
fused_copy_sfa = torch.ops.nanovllm_dsa.fused_copy_sfa.default
fused_copy_sfa_mtp = torch.ops.nanovllm_dsa.fused_copy_sfa_mtp.default
dsa_indexer_query_rope_inplace = torch.ops.nanovllm_dsa.dsa_indexer_query_rope_inplace.default
