"""IndexShare decode: owner layers select, shared layers reuse the selection.

GLM-5.2 runs the LightningIndexer in 21 of its 78 target layers.  Each
``full`` layer owns a group; the ``shared`` layers after it (up to the next
``full`` layer) keep their own KV payload but attend to the slots the owner
chose, and copy the owner's misses from their own DRAM cache into their own
HBM cache.

* :func:`glm52_indexer_types` -- the official schedule (reference
  nanovllm/config.py:26-33): layers 0-2 and every fourth layer from 6 are
  ``full``.
* :class:`IndexShareGroupManager` -- group topology with the reference's API
  and errors (nanovllm/engine/dsa_offload.py:324-474); without a schedule
  every layer is its own owner (GLM-5.1).
* :class:`IndexShareDecodeStep` -- one decode step over a stack of layers.
  An owner runs ``fused_li_manage(_mtp)`` into buffers it keeps per batch
  size; every member, the owner included, then runs ``fused_copy_sfa(_mtp)``
  (or ``scatter_copy`` + ``sparse_tail_attention(_mtp)``) on its own caches
  with those buffers (reference glm_mla.py:1336-1406, :1542-1611,
  :1752-1881).  A shared layer that runs before its owner in a step raises,
  as the reference does.  With ``prefetch=True`` (split path) the copies of
  a whole group run on a side stream as soon as its owner has selected, and
  each member's attention waits only for its own copy.

Nothing here allocates inside a step: the owner buffers are made once per
batch size, so a step can be captured in one HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Mapping, Sequence

import torch

from . import dsa_offload_ops as ops

TOPK = 2048
MTP_QUERIES = 4
MTP_UNION = MTP_QUERIES * TOPK


def glm52_indexer_types(num_hidden_layers: int) -> tuple[str, ...]:
    """``full`` for layers 0-2 and 6, 10, 14, ...; ``shared`` otherwise."""
    return tuple("full" if i < 3 or (i >= 6 and (i - 6) % 4 == 0) else "shared"
                 for i in range(int(num_hidden_layers)))


@dataclass(frozen=True)
class IndexShareGroup:
    """One owner layer and its members (the owner first)."""

    group_id: int
    owner_layer_idx: int
    member_layer_idxs: tuple[int, ...]


class IndexShareGroupManager:
    """Layer -> group / owner topology of an IndexShare schedule."""

    def __init__(self, num_hidden_layers: int, indexer_types: Sequence[str] | None = None) -> None:
        self.num_hidden_layers = int(num_hidden_layers)
        if indexer_types is None:
            groups = [IndexShareGroup(i, i, (i,)) for i in range(self.num_hidden_layers)]
        else:
            groups = self._from_types(tuple(str(t) for t in indexer_types))
        self._groups = tuple(groups)
        self._group_of: dict[int, int] = {}
        self._owner_of: dict[int, int] = {}
        for g in self._groups:
            for layer in g.member_layer_idxs:
                if layer in self._group_of:
                    raise ValueError(f"Layer {layer} appears in multiple IndexShare groups.")
                self._group_of[layer] = g.group_id
                self._owner_of[layer] = g.owner_layer_idx

    def _from_types(self, types: tuple[str, ...]) -> list[IndexShareGroup]:
        if len(types) != self.num_hidden_layers:
            raise ValueError("indexer_types length must match num_hidden_layers: "
                             f"got {len(types)}, expected {self.num_hidden_layers}.")
        members: list[list[int]] = []
        for layer, kind in enumerate(types):
            if kind == "full":
                members.append([layer])
            elif kind == "shared":
                if not members:
                    raise ValueError(f"Shared layer {layer} has no preceding full layer in indexer_types.")
                members[-1].append(layer)
            else:
                raise ValueError(f"Unknown indexer_type {kind!r} at layer {layer}; expected 'full' or 'shared'.")
        if not members:
            raise ValueError("indexer_types produced no IndexShare groups.")
        return [IndexShareGroup(gid, m[0], tuple(m)) for gid, m in enumerate(members)]

    @property
    def num_groups(self) -> int:
        return len(self._groups)

    @property
    def owner_layer_idxs(self) -> tuple[int, ...]:
        return tuple(g.owner_layer_idx for g in self._groups)

    @property
    def shared_layer_idxs(self) -> tuple[int, ...]:
        return tuple(i for i in range(self.num_hidden_layers) if not self.is_owner(i))

    def group_of(self, layer_idx: int) -> int:
        return self._group_of[int(layer_idx)]

    def owner_of(self, layer_idx: int) -> int:
        return self._owner_of[int(layer_idx)]

    def is_owner(self, layer_idx: int) -> bool:
        return self._owner_of[int(layer_idx)] == int(layer_idx)

    def is_shared(self, layer_idx: int) -> bool:
        return not self.is_owner(layer_idx)

    def group(self, group_id: int) -> IndexShareGroup:
        return self._groups[int(group_id)]

    def groups(self) -> tuple[IndexShareGroup, ...]:
        return self._groups

    def validate_layer(self, layer_idx: int) -> None:
        if int(layer_idx) not in self._group_of:
            raise IndexError(f"Layer {layer_idx} is not in any IndexShare group.")

    def __repr__(self) -> str:
        return (f"IndexShareGroupManager(layers={self.num_hidden_layers}, groups={self.num_groups}, "
                f"owners={self.owner_layer_idxs})")


@dataclass
class DsaLayerCaches:
    """One layer's persistent tensors.  KV caches are 4-D
    ``[blocks, 128, 1, 512 | 64]``; ``index_key_cache`` and
    ``cache_slots_pool`` belong to owner layers only."""

    hbm_k_rope: torch.Tensor
    hbm_kv_cache: torch.Tensor
    dram_k_rope: torch.Tensor
    dram_kv_cache: torch.Tensor
    index_key_cache: torch.Tensor | None = None
    cache_slots_pool: torch.Tensor | None = None


# Step-wide context (one block table for every layer, as in the model runner).
CONTEXT_FIELDS = ("index_block_table", "num_candidate_tokens", "num_cache_tokens", "req_pool_entries",
                  "hbm_block_table", "dram_block_table", "actual_seq_lengths_query", "actual_seq_lengths_kv")


class IndexShareDecodeStep:
    """Decode of one step over every layer of an IndexShare stack."""

    def __init__(self, groups: IndexShareGroupManager, layers: Sequence[DsaLayerCaches], *, mtp: bool = False,
                 fused: bool = True, prefetch: bool = False) -> None:
        if len(layers) != groups.num_hidden_layers:
            raise ValueError(f"expected {groups.num_hidden_layers} layers, got {len(layers)}")
        for owner in groups.owner_layer_idxs:
            if layers[owner].index_key_cache is None or layers[owner].cache_slots_pool is None:
                raise ValueError(f"owner layer {owner} needs index_key_cache and cache_slots_pool")
        if prefetch and fused:
            raise ValueError("prefetch copies on a side stream and attends with sparse_tail_attention: "
                             "pass fused=False")
        self.groups, self.layers, self.mtp, self.fused = groups, list(layers), bool(mtp), bool(fused)
        self.prefetch = bool(prefetch)
        self._copy_stream: torch.cuda.Stream | None = None
        self._events: list[torch.cuda.Event] = []
        self._outputs: dict[tuple[int, int], dict[str, torch.Tensor]] = {}
        self._selected: dict[int, int] = {}  # owner -> step id of its last selection
        self._step_id = 0

    def owner_outputs(self, owner: int, batch_size: int) -> dict[str, torch.Tensor]:
        """The owner's LIM buffers for ``batch_size`` (made on first use and
        reused, fixed addresses, as the reference's per-batch-size cache)."""
        key = (int(owner), int(batch_size))
        if key not in self._outputs:
            dev = self.layers[owner].hbm_kv_cache.device
            rows = batch_size * (MTP_QUERIES if self.mtp else 1)
            i32 = dict(dtype=torch.int32, device=dev)
            out = {"topk_src_ids": torch.full((rows, 1, TOPK), -1, **i32),
                   "topk_dst_slots": torch.full((rows, 1, TOPK), -1, **i32),
                   "miss_counts": torch.zeros(batch_size, **i32)}
            if self.mtp:
                out["miss_src_ids"] = torch.full((batch_size, MTP_UNION), -1, **i32)
                out["miss_dst_slots"] = torch.full((batch_size, MTP_UNION), -1, **i32)
            self._outputs[key] = out
        return self._outputs[key]

    def begin_step(self) -> None:
        self._step_id += 1

    def run_layer(self, layer_idx: int, ctx: Mapping[str, torch.Tensor], *, query_rope: torch.Tensor,
                  query: torch.Tensor, scale: float, attention_out: torch.Tensor,
                  query_index: torch.Tensor | None = None, index_weights: torch.Tensor | None = None) -> None:
        """Selection (owners), then copy + attention on this layer's caches."""
        self.groups.validate_layer(layer_idx)
        B = int(ctx["num_candidate_tokens"].shape[0])
        owner = self.groups.owner_of(layer_idx)
        if layer_idx == owner:
            self._select(owner, ctx, B, query_index, index_weights)
        elif self._selected.get(owner) != self._step_id:
            raise RuntimeError(f"Shared layer {layer_idx} decode ran before its owner's LIM update "
                               f"(owner {owner}, batch_size={B}).")
        if self.fused:
            self._attend(layer_idx, ctx, B, query_rope, query, scale, attention_out, fused=True)
        else:
            self._copy(layer_idx, ctx, B)
            self._attend(layer_idx, ctx, B, query_rope, query, scale, attention_out, fused=False)

    def _select(self, owner: int, ctx, B: int, query_index, index_weights) -> None:
        if query_index is None or index_weights is None:
            raise RuntimeError("LIDU decode requires indexer outputs.")
        out = self.owner_outputs(owner, B)
        lay = self.layers[owner]
        args = (query_index, index_weights, lay.index_key_cache, ctx["index_block_table"],
                ctx["num_candidate_tokens"], ctx["num_cache_tokens"], ctx["req_pool_entries"],
                lay.cache_slots_pool, out["topk_src_ids"], out["topk_dst_slots"])
        if self.mtp:
            ops.fused_li_manage_mtp(*args, out["miss_src_ids"], out["miss_dst_slots"], out["miss_counts"])
        else:
            ops.fused_li_manage(*args, out["miss_counts"])
        self._selected[owner] = self._step_id

    def _copy(self, layer_idx: int, ctx, B: int) -> None:
        """The owner's misses, this layer's DRAM -> this layer's HBM.  The copy
        takes 3-D cache views (reference glm_mla.py:1360-1363)."""
        out = self.owner_outputs(self.groups.owner_of(layer_idx), B)
        lay = self.layers[layer_idx]
        views = (lay.hbm_k_rope.squeeze(2), lay.hbm_kv_cache.squeeze(2), lay.dram_k_rope.squeeze(2),
                 lay.dram_kv_cache.squeeze(2))
        if self.mtp:
            ops.scatter_copy(out["miss_src_ids"], out["miss_dst_slots"], out["miss_counts"], ctx["hbm_block_table"],
                             ctx["dram_block_table"], *views)
        else:
            ops.scatter_copy(out["topk_src_ids"].view(B, TOPK), out["topk_dst_slots"].view(B, TOPK),
                             out["miss_counts"], ctx["hbm_block_table"], ctx["dram_block_table"], *views)

    def _attend(self, layer_idx: int, ctx, B: int, query_rope, query, scale, attention_out, *, fused: bool) -> None:
        out = self.owner_outputs(self.groups.owner_of(layer_idx), B)
        lay = self.layers[layer_idx]
        common = (query_rope, query, ctx["actual_seq_lengths_query"], ctx["actual_seq_lengths_kv"],
                  ctx["num_cache_tokens"], out["topk_dst_slots"])
        if fused:
            tail = (ctx["hbm_block_table"], ctx["dram_block_table"], lay.hbm_k_rope, lay.hbm_kv_cache,
                    lay.dram_k_rope, lay.dram_kv_cache, scale, attention_out)
            if self.mtp:
                ops.fused_copy_sfa_mtp(*common, out["topk_src_ids"], out["miss_src_ids"], out["miss_dst_slots"],
                                       out["miss_counts"], *tail)
            else:
                ops.fused_copy_sfa(*common, out["topk_src_ids"].view(B, TOPK), out["miss_counts"], *tail)
            return
        attend = ops.sparse_tail_attention_mtp if self.mtp else ops.sparse_tail_attention
        attend(*common, ctx["hbm_block_table"], lay.hbm_k_rope, lay.hbm_kv_cache, scale, attention_out)

    def step(self, ctx: Mapping[str, torch.Tensor], layer_inputs: Callable[[int], Mapping[str, object]]) -> None:
        """Run every layer in order; ``layer_inputs(i)`` gives layer i's
        keyword arguments of :meth:`run_layer` (owners add the indexer
        query and weights)."""
        missing = [f for f in CONTEXT_FIELDS if f not in ctx]
        if missing:
            raise ValueError(f"decode context is missing: {missing}")
        self.begin_step()
        if self.prefetch:
            self._step_prefetch(ctx, layer_inputs)
            return
        for i in range(self.groups.num_hidden_layers):
            self.run_layer(i, ctx, **layer_inputs(i))

    def _step_prefetch(self, ctx, layer_inputs) -> None:
        """Group prefetch: once an owner has selected, the copies of every
        member of its group (they depend only on the owner's buffers) run on a
        side stream, and each member's attention waits only for its own copy.
        The copy stream starts after the previous step's work on the current
        stream (the owner buffers and HBM slots it rewrites are free then) and
        rejoins the current stream at the end, so the step is one unit for a
        HIP graph capture."""
        B = int(ctx["num_candidate_tokens"].shape[0])
        dev = self.layers[0].hbm_kv_cache.device
        main = torch.cuda.current_stream(dev)
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=dev)
            self._events = [torch.cuda.Event() for _ in range(self.groups.num_hidden_layers + 1)]
        cs, ev = self._copy_stream, self._events
        cs.wait_stream(main)
        for g in self.groups.groups():
            kw = dict(layer_inputs(g.owner_layer_idx))
            self._select(g.owner_layer_idx, ctx, B, kw.pop("query_index", None), kw.pop("index_weights", None))
            ev[-1].record(main)
            cs.wait_event(ev[-1])
            with torch.cuda.stream(cs):
                for m in g.member_layer_idxs:
                    self._copy(m, ctx, B)
                    ev[m].record(cs)
            for m in g.member_layer_idxs:
                if m != g.owner_layer_idx:
                    kw = dict(layer_inputs(m))
                main.wait_event(ev[m])
                self._attend(m, ctx, B, kw["query_rope"], kw["query"], kw["scale"], kw["attention_out"], fused=False)
        main.wait_stream(cs)


__all__ = ["CONTEXT_FIELDS", "DsaLayerCaches", "IndexShareDecodeStep", "IndexShareGroup", "IndexShareGroupManager",
           "glm52_indexer_types"]
