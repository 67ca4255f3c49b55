"""HIP-graph replay of the DSA decode layer-step at fixed batch sizes.

The reference replays its whole stable decode step from captured graphs,
one per exact batch size, with every per-step input copied into
fixed-address buffers first (FullDecodeOnlyGraphManager and
FullDecodeGraphEntry, nanovllm/engine/full_decode_graph.py:33-57, :140-385,
:546-720).  This module does the same for the path this library owns: the
layer-step ``fused_li_manage(_mtp) -> fused_copy_sfa(_mtp)``.

* :func:`normalize_capture_sizes` / :func:`select_capture_size` keep the
  reference's rules (:33-57): sorted distinct positive sizes; a runtime batch
  runs in the smallest captured size that holds it.
* :class:`DsaLayerGraph` owns the static inputs and outputs of one batch
  size, captures the step once (after one eager warm-up that also sizes the
  operator workspaces) and replays it.  Rows past the runtime batch are
  padded so that every kernel skips them: no candidates, pool entry -1, no
  cache budget, zero visible length (LIM row guard, zero attention output).
  Tables narrower than the graph buffers are copied left-aligned and the
  rest zeroed (the reference's ``_copy_table``, :227-248).
* The KV caches, index keys and the LIDU pool are the caller's persistent
  tensors; their addresses are baked into the graph, as in the reference.

Inputs are copied with ordinary eager torch copies on the current stream
before each replay; nothing inside the graph is a memset.
"""

from __future__ import annotations

from typing import Iterable

import torch

from . import dsa_offload_ops as ops

MTP_QUERIES = 4
TOPK = 2048


def normalize_capture_sizes(values: Iterable[int]) -> tuple[int, ...]:
    """Validate, sort and deduplicate capture batch sizes (reference :33-45)."""
    sizes = tuple(sorted({int(v) for v in values}))
    if not sizes:
        raise ValueError("FULL_DECODE_ONLY requires at least one decode graph capture size. "
                         "Pass decode_graph_capture_sizes, for example (16,).")
    if sizes[0] <= 0:
        raise ValueError(f"Decode graph capture sizes must be positive, got {sizes}.")
    return sizes


def select_capture_size(real_batch_size: int, capture_sizes: Iterable[int]) -> int | None:
    """The smallest captured size that holds the batch (reference :48-56)."""
    for size in capture_sizes:
        if int(size) >= int(real_batch_size):
            return int(size)
    return None


# Per-request inputs and their padding value for rows past the runtime batch.
_ROW_INPUTS = {
    "num_candidate_tokens": 0,
    "num_cache_tokens": 0,
    "req_pool_entries": -1,
    "actual_seq_lengths_query": 1,
    "actual_seq_lengths_kv": 0,
}
_TABLES = ("index_block_table", "hbm_block_table", "dram_block_table")
# Per-query-row inputs (rows = requests x queries per request).
_QUERY_INPUTS = ("query_index", "index_weights", "query_rope", "query")


class DsaLayerGraph:
    """One captured DSA layer-step for ``batch_size`` requests."""

    def __init__(self, batch_size: int, *, index_key_cache: torch.Tensor, cache_slots_pool: torch.Tensor,
                 hbm_k_rope: torch.Tensor, hbm_kv_cache: torch.Tensor, dram_k_rope: torch.Tensor,
                 dram_kv_cache: torch.Tensor, hbm_block_columns: int, dram_block_columns: int, heads: int,
                 index_heads: int, scale: float, mtp: bool = False, dtype: torch.dtype = torch.bfloat16) -> None:
        if batch_size <= 0:
            raise ValueError(f"batch_size must be positive, got {batch_size}")
        # The LIM operators require the index table to span the pool row
        # (S_cap == table columns * 128).
        index_block_columns = int(cache_slots_pool.shape[1]) // 128
        dev = hbm_kv_cache.device
        B = int(batch_size)
        q = MTP_QUERIES if mtp else 1
        rows = B * q
        i32 = dict(dtype=torch.int32, device=dev)
        f16 = dict(dtype=dtype, device=dev)
        self.batch_size, self.mtp, self.scale = B, bool(mtp), float(scale)
        self.persistent = dict(index_key_cache=index_key_cache, cache_slots_pool=cache_slots_pool,
                               hbm_k_rope=hbm_k_rope, hbm_kv_cache=hbm_kv_cache, dram_k_rope=dram_k_rope,
                               dram_kv_cache=dram_kv_cache)
        self.inputs = {
            "query_index": torch.zeros(rows, index_heads, 128, **f16),
            "index_weights": torch.zeros(rows, index_heads, **f16),
            "query_rope": torch.zeros(rows, heads, 64, **f16),
            "query": torch.zeros(rows, heads, 512, **f16),
            "index_block_table": torch.zeros(B, index_block_columns, **i32),
            "hbm_block_table": torch.zeros(B, hbm_block_columns, **i32),
            "dram_block_table": torch.zeros(B, dram_block_columns, **i32),
        }
        for name, pad in _ROW_INPUTS.items():
            self.inputs[name] = torch.full((B,), pad, **i32)
        self.outputs = {
            "topk_src_ids": torch.full((rows, 1, TOPK), -1, **i32),
            "topk_dst_slots": torch.full((rows, 1, TOPK), -1, **i32),
            "miss_counts": torch.zeros(B, **i32),
            "attention_out": torch.zeros(rows, heads, 512, **f16),
        }
        if mtp:
            self.outputs["miss_src_ids"] = torch.full((B, MTP_QUERIES * TOPK), -1, **i32)
            self.outputs["miss_dst_slots"] = torch.full((B, MTP_QUERIES * TOPK), -1, **i32)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.real_batch = 0
        self.replay_count = 0

    # -- the captured step ----------------------------------------------------
    def _step(self) -> None:
        i, o, p = self.inputs, self.outputs, self.persistent
        lim = (i["query_index"], i["index_weights"], p["index_key_cache"], i["index_block_table"],
               i["num_candidate_tokens"], i["num_cache_tokens"], i["req_pool_entries"], p["cache_slots_pool"],
               o["topk_src_ids"], o["topk_dst_slots"])
        common = (i["query_rope"], i["query"], i["actual_seq_lengths_query"], i["actual_seq_lengths_kv"],
                  i["num_cache_tokens"], o["topk_dst_slots"])
        caches = (i["hbm_block_table"], i["dram_block_table"], p["hbm_k_rope"], p["hbm_kv_cache"], p["dram_k_rope"],
                  p["dram_kv_cache"], self.scale, o["attention_out"])
        if self.mtp:
            ops.fused_li_manage_mtp(*lim, o["miss_src_ids"], o["miss_dst_slots"], o["miss_counts"])
            ops.fused_copy_sfa_mtp(*common, o["topk_src_ids"], o["miss_src_ids"], o["miss_dst_slots"],
                                   o["miss_counts"], *caches)
        else:
            ops.fused_li_manage(*lim, o["miss_counts"])
            ops.fused_copy_sfa(*common, o["topk_src_ids"].view(self.batch_size, TOPK), o["miss_counts"], *caches)

    def capture(self) -> None:
        """Warm up eagerly on a side stream (sizes the operator workspaces),
        then capture the step.  The warm-up runs with every row padded, so
        it changes no pool row and copies nothing."""
        stream = torch.cuda.Stream(device=self.outputs["miss_counts"].device)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            self._step()
        stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self._step()
        torch.cuda.current_stream().wait_stream(stream)

    # -- per-step inputs --------------------------------------------------------
    def copy_runtime_inputs(self, **runtime: torch.Tensor) -> int:
        """Copy one step's inputs into the static buffers; returns the runtime
        batch.  Every name in ``_ROW_INPUTS``, ``_TABLES`` and
        ``_QUERY_INPUTS`` is required."""
        missing = [n for n in (*_ROW_INPUTS, *_TABLES, *_QUERY_INPUTS) if n not in runtime]
        if missing:
            raise ValueError(f"missing runtime inputs: {missing}")
        real = int(runtime["num_candidate_tokens"].shape[0])
        if real > self.batch_size:
            raise ValueError(f"runtime batch {real} exceeds the graph's batch size {self.batch_size}")
        q = MTP_QUERIES if self.mtp else 1
        for name, pad in _ROW_INPUTS.items():
            src = runtime[name]
            if src.shape != (real,):
                raise ValueError(f"{name} must be [{real}], got {tuple(src.shape)}")
            self.inputs[name][:real].copy_(src)
            self.inputs[name][real:].fill_(pad)
        for name in _TABLES:
            src, dst = runtime[name], self.inputs[name]
            if src.dim() != 2 or src.shape[0] != real:
                raise ValueError(f"{name} must be rank 2 with {real} rows, got {tuple(src.shape)}")
            if src.shape[1] > dst.shape[1]:
                raise ValueError(f"{name} is wider than its graph buffer: runtime={src.shape[1]}, "
                                 f"graph={dst.shape[1]}.")
            dst[:real, :src.shape[1]].copy_(src)
            dst[:real, src.shape[1]:].zero_()
            dst[real:].zero_()
        for name in _QUERY_INPUTS:
            src, dst = runtime[name], self.inputs[name]
            if src.shape[0] != real * q or src.shape[1:] != dst.shape[1:]:
                raise ValueError(f"{name} must be [{real * q}, {', '.join(map(str, dst.shape[1:]))}], "
                                 f"got {tuple(src.shape)}")
            dst[:real * q].copy_(src)
            dst[real * q:].zero_()
        self.real_batch = real
        return real

    def replay(self, **runtime: torch.Tensor) -> dict[str, torch.Tensor]:
        """Copy the inputs (when given), replay, and return views of the
        outputs for the runtime rows."""
        if self.graph is None:
            raise RuntimeError("the graph is not captured; call capture() first")
        if runtime:
            self.copy_runtime_inputs(**runtime)
        self.graph.replay()
        self.replay_count += 1
        real = self.real_batch
        q = MTP_QUERIES if self.mtp else 1
        out = {k: (v[:real] if k in ("miss_counts", "miss_src_ids", "miss_dst_slots") else v[:real * q])
               for k, v in self.outputs.items()}
        return out


__all__ = ["DsaLayerGraph", "normalize_capture_sizes", "select_capture_size"]
