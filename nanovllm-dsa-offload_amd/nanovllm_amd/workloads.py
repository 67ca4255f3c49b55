"""Seeded synthetic workloads for the DSA offload chain.

Builds the inputs of one target layer's stable decode step the way the
reference's op tests and perf scripts do (ut_ops/test_fused_li_manage_scatter.py,
ut_ops/test_fused_copy_sfa.py, ut_ops/test_fused_li_manage_perf.py:221-257):
paged bf16 index keys and latent KV with random block tables, an index query
with U(0,1) head weights, a persistent slot pool holding a previous
selection (so that 5-15% of this step's top-2048 miss), an HBM cache
consistent with that pool, DRAM caches in host-mapped memory, and the
attention query.

``guard=True`` makes the integer outputs well defined under any fp32
summation order: it computes float64 scores plus a per-token bound on the
fp32 reduction error, and while the top-2048 boundary (or the victim
boundary when C > 2048) is closer than the two tokens' bounds it halves the
index key of the token just outside (or inside) that boundary.  Halving a
bf16 row is exact and scales that token's score by exactly 1/2 (the score is
positively homogeneous in the key), so no other token moves.

Everything is generated on the CPU as torch tensors; ``to_device`` moves a
case to the GPU.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

BLOCK = 128
TOPK = 2048
CKV = 512
KPE = 64
IDX = 128
MTP_Q = 4

_ERR_UNIT = 2.0 ** -24 * 256  # fp32 reduction-order error per unit of sum |terms|


def _bf16(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return x.to(dtype)


_FILL_CHUNK = 1 << 22  # elements per independently seeded chunk of a parallel fill


def randn_fill(shape, seed: int, dtype: torch.dtype, threads: int | None = None) -> torch.Tensor:
    """N(0,1) values of ``shape`` rounded to ``dtype``, filled in parallel.

    The tensor is cut into chunks of 2^22 elements, each drawn from its own
    torch CPU generator seeded by (seed, chunk), so the result depends only
    on the shape and the seed, not on the thread count.  Full-size
    configurations hold gigabytes of latent KV; a single generator takes
    about a minute for cfg2's, a pool of threads a few seconds."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    out = torch.empty(shape, dtype=dtype)
    flat = out.view(-1)
    n = flat.numel()
    nchunks = (n + _FILL_CHUNK - 1) // _FILL_CHUNK

    def job(i: int) -> None:
        g = torch.Generator().manual_seed((int(seed) * 1000003 + i) & ((1 << 63) - 1))
        lo = i * _FILL_CHUNK
        hi = min(n, lo + _FILL_CHUNK)
        flat[lo:hi].copy_(torch.randn(hi - lo, generator=g))

    workers = max(1, min(16, threads or os.cpu_count() or 1, nchunks))
    if workers == 1:
        for i in range(nchunks):
            job(i)
    else:
        with ThreadPoolExecutor(workers) as ex:
            list(ex.map(job, range(nchunks)))
    return out


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float64).numpy()


@dataclass
class ChainCase:
    """Inputs (and shapes) of one LIM -> copy -> SFA layer step."""

    tensors: dict[str, torch.Tensor] = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    def __getitem__(self, key):
        return self.tensors[key]

    def to_device(self, device, host_mapped: bool = True) -> "ChainCase":
        """Copy to ``device``; DRAM caches go to host-mapped memory unless
        ``host_mapped`` is False (then plain HBM)."""
        out = {}
        for name, t in self.tensors.items():
            if name in ("dram_kv_cache", "dram_k_rope") and host_mapped:
                from .host_memory import host_mapped_pair

                gpu, cpu = host_mapped_pair(t.shape, t.dtype, device)
                cpu.copy_(t)
                out[name] = gpu
                out[name + "_host"] = cpu
            else:
                out[name] = t.to(device)
        return ChainCase(out, dict(self.meta))


def _topk_order(scores: np.ndarray, head: int | None = None) -> np.ndarray:
    """Token ids by descending score, ties to the lower id.  With ``head``,
    only the first ``head`` entries of that order (exact: every token tied
    with the head-th largest score takes part in the ordering)."""
    n = scores.shape[0]
    if head is None or head >= n:
        return np.lexsort((np.arange(n), -scores))
    thr = np.partition(scores, n - head)[n - head]  # the head-th largest score
    cand = np.nonzero(scores >= thr)[0]
    return cand[np.lexsort((cand, -scores[cand]))][:head]


def make_chain_case(
    batch: int,
    source_lens,
    cache_tokens,
    tails,
    *,
    index_heads: int = 32,
    attn_heads: int = 64,
    miss_frac=(0.05, 0.15),
    seed: int = 0,
    dtype: torch.dtype = torch.bfloat16,
    mtp: bool = False,
    guard: bool = True,
    extra_pool_rows: int = 1,
    query_scale: float = 1.0,
    structured_scores: bool = False,
    source_capacity: int | None = None,
    table_pad: int = -1,
    fast_fill: bool = False,
    structured_orders=None,
    miss_fracs=None,
) -> ChainCase:
    """One layer step.  ``source_lens`` / ``cache_tokens`` / ``tails`` are
    per-request lists (or scalars); source lengths are whole 128-token
    blocks.  ``mtp`` builds four index/attention queries per request.
    ``structured_scores`` uses the reference's closed-form index (score ==
    token id, ut_ops/test_fused_li_manage.py:146-173).

    ``source_capacity`` widens the index block table and the slot pool to
    that many tokens (a multiple of 128) instead of the longest source, as
    the model runner does: it sizes the pool and pads every block table to
    ceil(max_model_len / 128) columns (nanovllm/engine/model_runner.py:587-598,
    :747-752; max_model_len = 65536 by default, nanovllm/config.py:68).
    ``table_pad`` fills the block-table columns past a request's blocks (the
    runner pads with 0).  ``fast_fill`` draws the large N(0,1) tensors with
    :func:`randn_fill` (different values from the serial generator).
    ``structured_orders`` (with ``structured_scores``) gives each query row
    its own weights for the key's base-64 digits (see
    :func:`structured_query`), so that the rows select different sets.
    ``miss_fracs`` (one per request) replaces the draw from ``miss_frac``."""
    B = int(batch)
    as_list = lambda v: [int(x) for x in (v if hasattr(v, "__len__") else [v] * B)]  # noqa: E731
    N = as_list(source_lens)
    C = as_list(cache_tokens)
    T = as_list(tails)
    Q = MTP_Q if mtp else 1
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    fill_seed = [seed * 16 + 1]

    def randn(*shape) -> torch.Tensor:
        """A large N(0,1) tensor in ``dtype`` (serial generator unless fast_fill)."""
        if fast_fill:
            fill_seed[0] += 1
            return randn_fill(shape, fill_seed[0], dtype)
        return torch.randn(*shape, generator=g).to(dtype)

    cols = max(1, math.ceil(max(N) / BLOCK))
    if source_capacity is not None:
        if source_capacity % BLOCK or source_capacity < cols * BLOCK:
            raise ValueError(f"source_capacity {source_capacity} must be a multiple of {BLOCK} covering every source")
        cols = source_capacity // BLOCK
    cap = cols * BLOCK
    # ---- index keys, paged -------------------------------------------------
    nblk = [math.ceil(n / BLOCK) for n in N]
    total_idx = max(1, sum(nblk))
    perm = torch.randperm(total_idx, generator=g).to(torch.int32)
    index_table = torch.full((B, cols), table_pad, dtype=torch.int32)
    off = 0
    for b in range(B):
        index_table[b, : nblk[b]] = perm[off : off + nblk[b]]
        off += nblk[b]
    if structured_scores:
        keys = torch.zeros(total_idx, BLOCK, 1, IDX)
        for b in range(B):
            ids = torch.arange(nblk[b] * BLOCK)
            rows = keys[index_table[b, : nblk[b]].long()].view(-1, IDX)
            rows[:, 0] = (ids % 64).float()
            rows[:, 1] = ((ids // 64) % 64).float()
            rows[:, 2] = ((ids // 4096) % 64).float()
            rows[:, 3] = (ids // 262144).float()
            keys[index_table[b, : nblk[b]].long()] = rows.view(nblk[b], BLOCK, 1, IDX)
        key_cache = keys.to(dtype)
        orders = structured_orders if structured_orders is not None else [(1.0, 64.0, 4096.0, 262144.0)] * Q
        q_index = torch.stack([structured_query(orders[r % len(orders)], index_heads) for r in range(B * Q)])
        q_index = q_index.to(dtype)
        weights = torch.zeros(B * Q, index_heads)
        weights[:, 0] = 1.0
        weights = weights.to(dtype)
    else:
        key_cache = randn(total_idx, BLOCK, 1, IDX)
        q_index = torch.randn(B * Q, index_heads, IDX, generator=g).to(dtype)
        weights = torch.rand(B * Q, index_heads, generator=g).to(dtype)

    kc = key_cache.view(-1, IDX)  # physical rows

    def rows_of(b: int) -> torch.Tensor:
        n = N[b]
        t = torch.arange(n)
        return index_table[b, t // BLOCK].long() * BLOCK + (t % BLOCK)

    def scores_of(b: int, phys: torch.Tensor):
        if not guard:
            # unguarded (benchmark) inputs: float32 scores are enough to place the pool
            k32 = kc[phys].float()
            s = [(torch.relu(k32 @ q_index[b * Q + q].float().T) @ weights[b * Q + q].float()).double().numpy()
                 for q in range(Q)]
            return np.stack(s), np.zeros((Q, phys.numel()))
        k = _f64(kc[phys])
        s, e = [], []
        for q in range(Q):
            qq = _f64(q_index[b * Q + q])
            ww = _f64(weights[b * Q + q])
            dots = k @ qq.T
            s.append(np.maximum(dots, 0.0) @ ww)
            if guard:
                e.append(_ERR_UNIT * (np.abs(k) @ np.abs(qq).T) @ np.abs(ww))
            else:
                e.append(np.zeros_like(s[-1]))
        return np.stack(s), np.stack(e)

    pool_rows = B + extra_pool_rows
    pool = torch.full((pool_rows, cap), -777, dtype=torch.int32)
    pool_entries = torch.from_numpy(rng.permutation(pool_rows)[:B].astype(np.int32))
    miss_target = []
    halvings = 0
    cached_lists, slot_lists = [], []
    for b in range(B):
        phys = rows_of(b)
        s, e = scores_of(b, phys)
        n, c = N[b], C[b]
        active = n >= TOPK and c >= TOPK and c <= n if not mtp else (n >= TOPK and c > 0 and c >= min(n, 8192) and c <= n)
        # ---- top-k boundary guard --------------------------------------------
        if guard and active and not structured_scores:
            for _ in range(4 * n):
                changed = False
                for q in range(Q):
                    order = _topk_order(s[q], TOPK + 1)
                    if n <= TOPK:
                        continue
                    a, z = order[TOPK - 1], order[TOPK]
                    if s[q, a] - s[q, z] < e[q, a] + e[q, z] + 1e-12:
                        kc[phys[z]] = (kc[phys[z]].float() * 0.5).to(dtype)
                        s[:, z] *= 0.5
                        e[:, z] *= 0.5
                        halvings += 1
                        changed = True
                if not changed:
                    break
        pool[pool_entries[b]].fill_(-1)
        if not active:
            miss_target.append(0)
            cached_lists.append(np.zeros(0, np.int64))
            slot_lists.append(np.zeros(0, np.int64))
            continue
        sel_rows = [np.sort(_topk_order(s[q], TOPK)) for q in range(Q)]
        if mtp:
            seen = set()
            union = []
            for row in sel_rows:
                for t in row:
                    if int(t) not in seen:
                        seen.add(int(t))
                        union.append(int(t))
            union = np.asarray(union, np.int64)
        else:
            union = sel_rows[0]
        frac = rng.uniform(*miss_frac)
        if miss_fracs is not None:
            frac = float(miss_fracs[b])
        m = int(round(frac * union.size))
        m = max(0, min(m, union.size, n - c))
        miss_target.append(m)
        misses = rng.choice(union, size=m, replace=False) if m else np.zeros(0, np.int64)
        in_union = np.zeros(n, bool)
        in_union[union] = True
        is_miss = np.zeros(n, bool)
        is_miss[misses] = True
        hits = union[~is_miss[union]]
        need = c - hits.size
        smax = s.max(axis=0)
        outside = np.nonzero(~in_union)[0]
        # fillers: previously selected tokens just outside this step's union
        outside_rank = outside[np.argsort(-smax[outside], kind="stable")]
        pool_sz = min(outside_rank.size, max(need, 4 * c))
        fillers = rng.choice(outside_rank[:pool_sz], size=need, replace=False) if need else np.zeros(0, np.int64)
        # ---- victim boundary guard (only when the victim set is not forced) --
        if guard and m > 0 and fillers.size > m and not structured_scores:
            emax = e.max(axis=0)
            for _ in range(4 * fillers.size):
                order = fillers[np.lexsort((fillers, smax[fillers]))]
                lo, hi = order[m - 1], order[m]
                if smax[hi] - smax[lo] >= emax[lo] + emax[hi] + 1e-12:
                    break
                kc[phys[lo]] = (kc[phys[lo]].float() * 0.5).to(dtype)
                s[:, lo] *= 0.5
                e[:, lo] *= 0.5
                smax[lo] *= 0.5
                emax[lo] *= 0.5
                halvings += 1
        cached = np.concatenate([hits, fillers]).astype(np.int64)
        slots = rng.permutation(c).astype(np.int64)
        pool[pool_entries[b], torch.from_numpy(cached)] = torch.from_numpy(slots.astype(np.int32))
        cached_lists.append(cached)
        slot_lists.append(slots)

    # ---- latent KV: DRAM (full prompt) and HBM (C slots + tail) ------------------
    dram_table = torch.full((B, cols), table_pad, dtype=torch.int32)
    dperm = torch.randperm(total_idx, generator=g).to(torch.int32)
    off = 0
    for b in range(B):
        dram_table[b, : nblk[b]] = dperm[off : off + nblk[b]]
        off += nblk[b]
    dram_ckv = randn(total_idx, BLOCK, CKV)
    dram_kpe = randn(total_idx, BLOCK, KPE)
    hlen = [C[b] + T[b] for b in range(B)]
    hblk = [max(1, math.ceil(h / BLOCK)) for h in hlen]
    hcols = max(hblk)
    total_h = sum(hblk)
    hperm = torch.randperm(total_h, generator=g).to(torch.int32)
    hbm_table = torch.full((B, hcols), table_pad, dtype=torch.int32)
    off = 0
    for b in range(B):
        hbm_table[b, : hblk[b]] = hperm[off : off + hblk[b]]
        off += hblk[b]
    hbm_ckv = randn(total_h, BLOCK, 1, CKV)
    hbm_kpe = randn(total_h, BLOCK, 1, KPE)
    hc = hbm_ckv.view(-1, CKV)
    hk = hbm_kpe.view(-1, KPE)
    dc = dram_ckv.view(-1, CKV)
    dk = dram_kpe.view(-1, KPE)
    for b in range(B):
        cached, slots = cached_lists[b], slot_lists[b]
        if cached.size == 0:
            continue
        st = torch.from_numpy(slots)
        hrow = hbm_table[b, st // BLOCK].long() * BLOCK + st % BLOCK
        ct = torch.from_numpy(cached)
        drow = dram_table[b, ct // BLOCK].long() * BLOCK + ct % BLOCK
        hc[hrow] = dc[drow]
        hk[hrow] = dk[drow]

    R = B * Q
    q_attn = (torch.randn(R, attn_heads, CKV, generator=g) * query_scale).to(dtype)
    q_rope = (torch.randn(R, attn_heads, KPE, generator=g) * query_scale).to(dtype)
    tensors = {
        "query_index": q_index,
        "index_weights": weights,
        "index_key_cache": key_cache,
        "index_block_table": index_table,
        "num_candidate_tokens": torch.tensor(N, dtype=torch.int32),
        "num_cache_tokens": torch.tensor(C, dtype=torch.int32),
        "req_pool_entries": pool_entries,
        "cache_slots_pool": pool,
        "query": q_attn,
        "query_rope": q_rope,
        "actual_seq_lengths_query": torch.arange(Q, R + 1, Q, dtype=torch.int32)[:B]
        if Q > 1
        else torch.arange(1, B + 1, dtype=torch.int32),
        "actual_seq_lengths_kv": torch.tensor(hlen, dtype=torch.int32),
        "hbm_block_table": hbm_table,
        "dram_block_table": dram_table,
        "hbm_kv_cache": hbm_ckv,
        "hbm_k_rope": hbm_kpe,
        "dram_kv_cache": dram_ckv,
        "dram_k_rope": dram_kpe,
    }
    # caller-owned outputs
    tensors["topk_src_ids"] = torch.full((R, 1, TOPK), -1, dtype=torch.int32)
    tensors["topk_dst_slots"] = torch.full((R, 1, TOPK), -1, dtype=torch.int32)
    tensors["miss_counts"] = torch.full((B,), -1, dtype=torch.int32)
    if mtp:
        tensors["miss_src_ids"] = torch.full((B, 8192), -1, dtype=torch.int32)
        tensors["miss_dst_slots"] = torch.full((B, 8192), -1, dtype=torch.int32)
    tensors["attention_out"] = torch.zeros(R, attn_heads, CKV, dtype=dtype)
    meta = {
        "batch": B,
        "source_lens": N,
        "cache_tokens": C,
        "tails": T,
        "mtp": mtp,
        "queries": Q,
        "miss_target": miss_target,
        "halvings": halvings,
        "scale": 1.0 / math.sqrt(CKV + KPE),
        "dtype": dtype,
    }
    return ChainCase(tensors, meta)


def structured_query(order, heads: int = 32) -> torch.Tensor:
    """One index query row over the closed-form keys of
    :func:`make_chain_case` (``structured_scores``: a token's key holds its
    base-64 digits t % 64, (t >> 6) % 64, (t >> 12) % 64, t >> 18 in dims
    0-3; ut_ops/test_fused_li_manage.py:146-173): head 0 weights the digits
    by ``order``, every other head is zero.  With the weights (1, 0, ...)
    the score is sum_i order[i] * digit_i, an integer below 2^24 whenever
    the weights are distinct powers of 64: exact in fp32 under any
    summation order, and distinct for distinct tokens."""
    q = torch.zeros(heads, IDX)
    q[0, :4] = torch.tensor([float(x) for x in order])
    return q


# Digit weights of the structured MTP3 drift queries: the six orders of the
# three low digits (the fourth digit is 0 below 262144 tokens).
STRUCTURED_ORDERS = {
    "t": (1.0, 64.0, 4096.0, 0.0), "d0": (4096.0, 1.0, 64.0, 0.0), "d1": (1.0, 4096.0, 64.0, 0.0),
    "d0d2": (64.0, 1.0, 4096.0, 0.0), "d1d0": (64.0, 4096.0, 1.0, 0.0), "d0d1": (4096.0, 64.0, 1.0, 0.0),
}


def make_structured_drift_case(batch: int, source_lens, cache_tokens, tails, orders_a, orders_b, *, mtp: bool = True,
                               seed: int = 0, dtype: torch.dtype = torch.bfloat16, fast_fill: bool = False,
                               source_capacity: int | None = None) -> ChainCase:
    """Two alternating index queries over the closed-form index: query row
    j of ``query_index`` weights the key digits by ``orders_a[j]``, of
    ``query_index_b`` by ``orders_b[j]`` (:func:`structured_query`).  The
    scores are exact integers, so every step's selection and victims are
    the same under any fp32 summation order without a guard (victim-key ties
    are exact too, and go to the lower slot by the canonical rule).  The pool
    starts with ``query_index``'s union cached (plus the highest-scoring
    other tokens up to C); the HBM cache matches it."""
    case = make_chain_case(batch, source_lens, cache_tokens, tails, miss_frac=(0.0, 0.0), seed=seed, dtype=dtype,
                           guard=False, mtp=mtp, structured_scores=True, structured_orders=list(orders_a),
                           fast_fill=fast_fill, source_capacity=source_capacity)
    Q = case.meta["queries"]
    B = case.meta["batch"]
    case.tensors["query_index_b"] = torch.stack(
        [structured_query(orders_b[r % Q], case.tensors["query_index"].shape[1]) for r in range(B * Q)]).to(dtype)
    return case


RUNNER_CAPACITY = 65536  # default max_model_len (nanovllm/config.py:68), in tokens


def caller_layout(t: dict, capacity: int = RUNNER_CAPACITY, pad: int = 0) -> dict:
    """The same step with the model runner's table layout: index, DRAM and
    HBM block tables padded to ``capacity``/128 columns with ``pad`` (the
    runner pads with 0, nanovllm/engine/model_runner.py:747-752; columns past
    a request's blocks that held -1 get ``pad`` too) and the slot pool
    ``capacity`` wide (model_runner.py:587-598); new pool columns of a
    request's row hold -1, of other rows -777.  Works on CPU or GPU tensors;
    returns a new dict with new tensors for the widened ones."""
    out = dict(t)
    cols = capacity // BLOCK
    for name in ("index_block_table", "dram_block_table", "hbm_block_table"):
        old = t[name]
        if old.shape[1] > cols:
            raise ValueError(f"{name} is wider than {capacity} tokens")
        new = torch.full((old.shape[0], cols), pad, dtype=old.dtype, device=old.device)
        keep = old.clone()
        keep[keep < 0] = pad
        new[:, :old.shape[1]] = keep
        out[name] = new
    pool = t["cache_slots_pool"]
    wide = torch.full((pool.shape[0], capacity), -777, dtype=pool.dtype, device=pool.device)
    wide[:, :pool.shape[1]] = pool
    wide[t["req_pool_entries"].long(), pool.shape[1]:] = -1
    out["cache_slots_pool"] = wide
    return out


def baseline_config(index: int, seed: int = 0, dtype: torch.dtype = torch.bfloat16, guard: bool = False,
                    source_capacity: int | None = None, table_pad: int = -1, fast_fill: bool = True) -> ChainCase:
    """The configurations of BASELINE.json ``configs`` (0..3) at full size.

    cfg0: bs=1, 20480-token prompt, tail 37, C=2048.
    cfg1: bs=24, 32768-token prompts, tails U[1,127], miss 5-15%, C=2048.
    cfg2: bs=64, prompts U[20K,64K] (whole blocks), C=2048 (fused path).
    cfg3: MTP3, bs=16 x 4 queries, 48K prompts, C=8192.

    ``source_capacity`` / ``table_pad`` give the caller's table layout (see
    :func:`make_chain_case`); by default the tables are as wide as the
    longest source.
    """
    rng = np.random.default_rng(1000 + index)
    kw = dict(seed=seed, dtype=dtype, guard=guard, source_capacity=source_capacity, table_pad=table_pad,
              fast_fill=fast_fill)
    if index == 0:
        return make_chain_case(1, 20480, 2048, 37, miss_frac=(0.1, 0.1), **kw)
    if index == 1:
        tails = rng.integers(1, 128, size=24)
        return make_chain_case(24, 32768, 2048, tails, **kw)
    if index == 2:
        lens = (rng.integers(20480, 65536 + 1, size=64) // BLOCK) * BLOCK
        tails = rng.integers(1, 128, size=64)
        return make_chain_case(64, lens, 2048, tails, **kw)
    if index == 3:
        tails = rng.integers(4, 128, size=16)
        return make_chain_case(16, 49152, 8192, tails, mtp=True, **kw)
    raise ValueError(f"no baseline config {index}")


def _torch_scores(keys: torch.Tensor, q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return torch.relu(keys @ q.T) @ w


def make_drift_case(
    batch: int,
    source_lens,
    cache_tokens,
    tails,
    *,
    miss_frac=(0.05, 0.15),
    seed: int = 0,
    dtype: torch.dtype = torch.bfloat16,
    index_heads: int = 32,
    attn_heads: int = 64,
    calib_device=None,
    mtp: bool = False,
    guard: bool = False,
    guard_steps: int = 8,
    guard_first: str = "query_index_b",
    fast_fill: bool = False,
    source_capacity: int | None = None,
) -> ChainCase:
    """Steady-state decode workload: two index queries that alternate.

    Adds a second index query ``query_index_b`` per request (MTP3: per query
    row, one perturbation size shared by a request's four rows), a
    perturbation of ``query_index`` calibrated (bisection on the
    perturbation size) so that its top-2048 set (MTP3: the union of the four
    rows' sets) differs from the first query's by the request's target miss
    fraction drawn from ``miss_frac``.  The pool starts with the first
    query's top-C cached; alternating the two queries step after step then
    makes every step miss ~that fraction, with the HBM cache kept consistent
    by the copies themselves -- no state restore between steps.

    ``guard=True`` makes every step of ``guard_steps`` alternating steps
    (``guard_first`` first, starting from the initial pool) well defined
    under any fp32 summation order: see :func:`guard_alternating_steps`
    (for MTP3 cases, whose eight rows make its halvings cascade, see
    :func:`make_structured_drift_case`).
    """
    case = make_chain_case(batch, source_lens, cache_tokens, tails, miss_frac=(0.0, 0.0), seed=seed, dtype=dtype,
                           guard=False, index_heads=index_heads, attn_heads=attn_heads, mtp=mtp,
                           fast_fill=fast_fill, source_capacity=source_capacity)
    t = case.tensors
    B = case.meta["batch"]
    Q = MTP_Q if mtp else 1
    rng = np.random.default_rng(seed + 7)
    g = torch.Generator().manual_seed(seed + 7)
    dev = torch.device(calib_device) if calib_device is not None else torch.device("cpu")
    kc = t["index_key_cache"].view(-1, IDX).to(dev).float()
    qa = t["query_index"].to(dev).float()
    w = t["index_weights"].to(dev).float()
    table = t["index_block_table"].to(dev)
    qb = torch.empty_like(t["query_index"])
    achieved = []

    def selected(keys, qrows, wrows, n):
        mask = torch.zeros(n, dtype=torch.bool, device=dev)
        for j in range(Q):
            mask[torch.topk(_torch_scores(keys, qrows[j], wrows[j]), TOPK).indices] = True
        return mask

    for b in range(B):
        n = case.meta["source_lens"][b]
        rows = slice(b * Q, b * Q + Q)
        if n <= TOPK or case.meta["cache_tokens"][b] < TOPK:
            qb[rows] = t["query_index"][rows]
            achieved.append(0.0)
            continue
        tok = torch.arange(n, device=dev)
        keys = kc[table[b, tok // BLOCK].long() * BLOCK + tok % BLOCK]
        in_a = selected(keys, qa[rows], w[rows], n)
        eps = torch.randn(qa[rows].shape, generator=g).to(dev)
        target = rng.uniform(*miss_frac)
        lo, hi = 0.0, 2.0
        best = (1.0, qa[rows].to(dtype), 0.0)
        for _ in range(14):
            mid = 0.5 * (lo + hi)
            cand = (qa[rows] + mid * eps).to(dtype)
            in_b = selected(keys, cand.float(), w[rows], n)
            frac = float((in_b & ~in_a).sum()) / float(in_b.sum())
            if abs(frac - target) < abs(best[0] - target):
                best = (frac, cand, mid)
            if frac < target:
                lo = mid
            else:
                hi = mid
        qb[rows] = best[1].cpu()
        achieved.append(best[0])
    t["query_index_b"] = qb
    case.meta["drift_miss_frac"] = achieved
    case.meta["guard_steps"] = 0
    if guard:
        names = ("query_index_b", "query_index")
        if guard_first not in names:
            raise ValueError(f"guard_first must be one of {names}")
        names = names if guard_first == names[0] else names[::-1]
        case.meta["halvings"] += guard_alternating_steps(case, names, guard_steps)
        case.meta["guard_steps"] = guard_steps
        case.meta["guard_first"] = guard_first
    return case


class _RowWindow:
    """The ``TOPK + window`` highest-scoring tokens of one query row in
    descending order (ties to the lower token), kept up to date while tokens
    are halved: a halved token leaves the window and re-enters at its new
    place only if it still ranks inside it.  The order of the other tokens
    does not change, so no re-sort is needed."""

    def __init__(self, scores: np.ndarray, window: int = 1024) -> None:
        self.s = scores
        self.window = window
        self.refresh()

    def refresh(self) -> None:
        self.top = [int(x) for x in _topk_order(self.s, TOPK + self.window)]
        self.member = set(self.top)

    def halved(self, tok: int) -> None:
        if tok not in self.member:
            return
        self.top.remove(tok)
        self.member.discard(tok)
        last = self.top[-1]
        v = self.s[tok]
        if v > self.s[last] or (v == self.s[last] and tok < last):
            lo, hi = 0, len(self.top)
            while lo < hi:  # first position whose token ranks below tok
                mid = (lo + hi) // 2
                u = self.top[mid]
                if self.s[u] > v or (self.s[u] == v and u < tok):
                    lo = mid + 1
                else:
                    hi = mid
            self.top.insert(lo, tok)
            self.member.add(tok)
        if len(self.top) < TOPK + 2:
            self.refresh()


def guard_alternating_steps(case: ChainCase, query_names, steps: int, max_halvings: int | None = None) -> int:
    """Make ``steps`` consecutive LIM steps well defined under any fp32
    summation order, step i using ``query_names[i % len(query_names)]``,
    the slot pool carried from step to step (no restore), starting from the
    case's pool.

    With float64 scores and a per-token bound on the fp32 reduction error
    (the bound of :func:`make_chain_case`), it requires:

    * for every query row of every query tensor, a gap larger than the two
      tokens' bounds between the 2048th and 2049th largest scores (these do
      not depend on the carried state);
    * at every step where the victims are not forced (more cached tokens
      outside the selection than misses), a gap larger than the bounds
      between the last victim and the first kept token by the victim key
      (MTP3: the largest of the step's four row scores), the cached set
      followed through the steps.

    Where a gap is too small it halves the index key of the token just
    outside the selection (or the last victim), which scales that token's
    scores by exactly 1/2 for every query, and checks again.  The slots need
    no guard: pairing victims with misses is an integer rule.

    The error bound spans about ten score spacings at a 32K-token boundary,
    so a boundary is cleared by halving the ~10 tokens below it.  With one
    row per query tensor (MTP0) the two tensors' boundaries sit among the
    same tokens and that is all.  With eight rows (MTP3) a halved token is
    often inside another row's selection, whose boundary then moves by one
    and needs its own ~10 halvings: the halvings cascade through the whole
    prompt, and the limit (2n halvings per request) raises an error.
    Returns the number of halvings."""
    t = case.tensors
    B = case.meta["batch"]
    Q = case.meta["queries"]
    mtp = case.meta["mtp"]
    dtype = t["index_key_cache"].dtype
    kc = t["index_key_cache"].view(-1, IDX)
    table = t["index_block_table"]
    pool = t["cache_slots_pool"]
    halvings = 0
    for b in range(B):
        n, c = case.meta["source_lens"][b], case.meta["cache_tokens"][b]
        active = (n > TOPK and c >= TOPK and c <= n) if not mtp else (n > TOPK and c >= min(n, 8192) and c <= n)
        if not active:
            continue
        limit = max_halvings if max_halvings is not None else 2 * n
        tok = torch.arange(n)
        phys = table[b, tok // BLOCK].long() * BLOCK + tok % BLOCK
        k = _f64(kc[phys])
        ka = np.abs(k)
        s, e, win = {}, {}, []
        for name in query_names:
            qq = _f64(t[name][b * Q:(b + 1) * Q])      # [Q, H, 128]
            ww = _f64(t["index_weights"][b * Q:(b + 1) * Q])
            s[name] = np.stack([np.maximum(k @ qq[j].T, 0.0) @ ww[j] for j in range(Q)])
            e[name] = np.stack([_ERR_UNIT * (ka @ np.abs(qq[j]).T) @ np.abs(ww[j]) for j in range(Q)])
            win += [(name, j, _RowWindow(s[name][j])) for j in range(Q)]
        row = pool[t["req_pool_entries"][b]].numpy()[:n]
        cached0 = (row >= 0) & (row < c)
        count = [0]

        def halve(z: int) -> None:
            if count[0] >= limit:
                raise RuntimeError(f"request {b}: no well-defined step sequence after {limit} halvings")
            kc[phys[z]] = (kc[phys[z]].float() * 0.5).to(dtype)
            for name in query_names:
                s[name][:, z] *= 0.5
                e[name][:, z] *= 0.5
            for _, _, w in win:
                w.halved(z)
            count[0] += 1

        while True:
            changed = True
            while changed:
                changed = False
                for name, j, w in win:
                    while True:
                        a, z = w.top[TOPK - 1], w.top[TOPK]
                        if s[name][j, a] - s[name][j, z] >= e[name][j, a] + e[name][j, z] + 1e-12:
                            break
                        halve(z)
                        changed = True
            union = {name: np.zeros(n, bool) for name in query_names}
            for name, _, w in win:
                union[name][np.asarray(w.top[:TOPK])] = True
            bad = None
            cached = cached0.copy()
            for step in range(steps):
                name = query_names[step % len(query_names)]
                sel = union[name]
                misses = np.nonzero(sel & ~cached)[0]
                cand = np.nonzero(cached & ~sel)[0]
                m = misses.size
                if 0 < m < cand.size:
                    smax, emax = s[name].max(axis=0), e[name].max(axis=0)
                    order = cand[np.lexsort((cand, smax[cand]))]
                    lo, hi = order[m - 1], order[m]
                    if smax[hi] - smax[lo] < emax[lo] + emax[hi] + 1e-12:
                        bad = int(lo)
                        break
                    victims = order[:m]
                else:
                    victims = cand[:m]
                cached[victims] = False
                cached[misses] = True
            if bad is None:
                break
            halve(bad)
        halvings += count[0]
    return halvings
