"""CPU oracle of the DSA stable-decode offload chain — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the
timed CPU baseline).  The product path (``nanovllm_amd``) never imports,
calls or falls back to it.

It restates, in numpy, the semantics of the seven reference operators:

* ``index_scores`` / ``topk_mask`` / ``lim_manage_row`` / ``fused_li_manage``
  — reference README_ops.md:19-33, ut_ops/FUSED_LI_MANAGE_BEHAVIOR.md:15-25,
  ops/fused_li_manage/op_kernel/fused_li_manage_service_cube.h:351 (ReLU),
  fused_li_manage_vector.h:97-167 (weights x heads reduce),
  fused_li_manage_vector.h:408-416 (miss-first / descending-slot hit order),
  fused_li_manage_kernel.h:261-290 (row guards);
* ``fused_li_manage_mtp`` — README_ops.md:35-51,
  ut_ops/test_fused_li_manage_mtp.py:127-137 (ordered union), :789-960,
  ops/fused_li_manage_mtp/op_kernel/fused_li_manage_mtp_kernel.h:218-233;
* ``scatter_copy`` — ut_ops/test_scatter_copy.py:125-147 (``apply_reference``),
  ops/kvcache_scatter_copy/op_kernel/kvcache_scatter_copy_kernel.h:141-177;
* ``sparse_tail_attention(_mtp)`` — ut_ops/test_sparse_tail_attention.py:190-216,
  ut_ops/test_sparse_tail_attention_mtp.py:314-327,
  ops/sparse_tail_attention/op_kernel/nanovllm_sparse_tail_attention_kernel_mla.h:325-353;
* ``fused_copy_sfa(_mtp)`` — the composition scatter_copy -> attention
  (ut_ops/test_fused_copy_sfa.py:453-497, README_ops.md:99-141);
* ``initialize_lidu_row(_shared)`` — the first-decode top-C initialisation
  and its IndexShare copy (nanovllm/models/dsa_offload_ops.py:251-411);
* ``persist_blocks`` / ``finalize_prefill_pool_row`` — the prefill -> DRAM
  hand-over of one layer (nanovllm/models/glm_mla.py:850-891).

Where the reference leaves a choice implementation-defined (victim choice —
a hash-seeded partial scan in fused_li_manage_service_vector.h:72-81,
:669-751 — and in-row order within the miss and hit segments,
FUSED_LI_MANAGE_BEHAVIOR.md:25), this oracle fixes the canonical rule the
HIP kernels implement:

* selection ties at the top-2048 threshold go to the lower token id;
* victims are the |M| non-hit slots with the lowest score (a slot held by no
  candidate token ranks first), ties to the lower slot; victim slots are
  paired in ascending order with the misses (MTP0: ascending token id;
  MTP3: ordered-union order);
* an attention key whose slot is negative, >= the visible length, or does
  not resolve through the block table is left out of the softmax;
* first-decode init gives slot i to the i-th smallest selected token;
* an index block-table entry that names no key block scores its tokens
  -FLT_MAX (the reference reads that memory unchecked).

Parity unpinned (no reference test or vector fixes them): the reference's own
victim choice and in-row order where they differ from the rules above, and
the slot order of ``initialize_lidu_row`` (the reference takes
``torch.topk(..., sorted=False)``, whose order is implementation-defined).
Every other output of these functions is pinned by tests/test_oracle.py,
tests/test_lidu_init.py and tests/test_golden.py.

Scores are computed in float64; the attention golden in float64 (and
optionally float32 like the reference test).  16-bit tensors are passed as
their raw uint16 bit patterns plus a dtype name ("bf16" or "f16").
"""

from __future__ import annotations

import numpy as np

BLOCK = 128
TOPK = 2048
CKV = 512
KPE = 64
IDX = 128
MTP_Q = 4
UNION_CAP = TOPK * MTP_Q
MAX_CACHE_TOKENS = (1 << 14) - 1
MAX_ACTUAL_SEQ_LEN = (1 << 21) - 1


# --------------------------------------------------------------------------
# 16-bit float codecs
def bits_to_f32(bits: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Raw uint16/int16 bit patterns -> float32 values."""
    u = np.asarray(bits).view(np.uint16)
    if dtype == "bf16":
        return (u.astype(np.uint32) << 16).view(np.float32)
    if dtype == "f16":
        return u.view(np.float16).astype(np.float32)
    raise ValueError(dtype)


def f32_to_bits(x: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """float32 -> 16-bit patterns, round to nearest even."""
    x = np.atleast_1d(np.asarray(x, dtype=np.float32))
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# --------------------------------------------------------------------------
# LightningIndexer scores and top-k
def index_scores(query: np.ndarray, weights: np.ndarray, keys: np.ndarray) -> np.ndarray:
    """s[t] = sum_h w[h] * max(0, q[h] . k[t]) in float64.

    query [H, 128], weights [H], keys [T, 128] (float arrays).
    Reference: fused_li_manage_service_cube.h:351 (ReLU on the cube result),
    fused_li_manage_vector.h:97-167 (scale by head weight, reduce heads).
    """
    dots = np.asarray(keys, np.float64) @ np.asarray(query, np.float64).T  # [T, H]
    return np.maximum(dots, 0.0) @ np.asarray(weights, np.float64)


def gather_rows(cache: np.ndarray, table_row: np.ndarray, n: int) -> np.ndarray:
    """Logical rows [0, n) of a paged cache [blocks, 128, ..., D] -> [n, D]."""
    cols = np.arange(n) // BLOCK
    offs = np.arange(n) % BLOCK
    phys = np.asarray(table_row)[cols].astype(np.int64)
    flat = cache.reshape(cache.shape[0], BLOCK, -1)
    return flat[phys, offs]


def index_scores_paged(query: np.ndarray, weights: np.ndarray, key_cache: np.ndarray, table_row: np.ndarray,
                       n: int, score_fn=None) -> np.ndarray:
    """Scores of logical tokens [0, n) whose keys sit in a paged cache.

    A block-table entry that names no block (negative, or >= the cache's
    block count) gives its tokens the score -FLT_MAX, below every real
    score and above a free slot's victim key (-inf).  The reference reads
    such an entry's memory unchecked (fused_li_manage_service_cube.h:217);
    the guard is this build's own, and the HIP score kernels write the same
    value.
    """
    table_row = np.asarray(table_row)
    blocks = key_cache.shape[0]
    phys = table_row[np.arange(n) // BLOCK].astype(np.int64)
    bad = (phys < 0) | (phys >= blocks)
    safe = table_row.copy()
    safe[(safe < 0) | (safe >= blocks)] = 0
    keys = gather_rows(key_cache, safe, n)
    s = (score_fn or index_scores)(query, weights, keys)
    s[bad] = -float(np.finfo(np.float32).max)
    return s


def topk_mask(scores: np.ndarray, k: int) -> np.ndarray:
    """Boolean mask of the k largest scores; ties go to the lower index."""
    n = scores.shape[0]
    order = np.lexsort((np.arange(n), -np.asarray(scores, np.float64)))
    mask = np.zeros(n, dtype=bool)
    mask[order[:k]] = True
    return mask


def _victim_slots(c: int, m: int, slot_state: np.ndarray, slot_key: np.ndarray) -> np.ndarray:
    """The m non-hit slots of [0, c) with the smallest key (free slots first,
    then ascending key, ties ascending slot), returned in ascending slot order."""
    if m <= 0:
        return np.zeros(0, dtype=np.int64)
    slots = np.arange(c)
    nonhit = slot_state != 1
    keys = np.where(slot_state == 0, -np.inf, slot_key)
    cand = slots[nonhit]
    order = np.lexsort((cand, keys[nonhit]))
    chosen = cand[order[:m]]
    return np.sort(chosen)


def _slot_tables(pool_row: np.ndarray, n: int, c: int, selected: np.ndarray, key: np.ndarray):
    slots = np.asarray(pool_row[:n]).astype(np.int64)
    cached = (slots >= 0) & (slots < c)
    state = np.zeros(c, dtype=np.int8)
    tok = np.full(c, -1, dtype=np.int64)
    skey = np.zeros(c, dtype=np.float64)
    hit_t = np.nonzero(cached & selected)[0]
    cand_t = np.nonzero(cached & ~selected)[0]
    state[slots[hit_t]] = 1
    tok[slots[hit_t]] = hit_t
    state[slots[cand_t]] = 2
    tok[slots[cand_t]] = cand_t
    skey[slots[cand_t]] = key[cand_t]
    return slots, cached, state, tok, skey


def lim_row_valid(n: int, c: int, r: int, cap: int, pool_rows: int) -> bool:
    """MTP0 row guard (fused_li_manage_kernel.h:261-290, plus C <= 16383)."""
    return (0 < n <= MAX_ACTUAL_SEQ_LEN and n <= cap and 0 <= r < pool_rows and c >= TOPK
            and c <= MAX_CACHE_TOKENS and c <= n)


def lim_mtp_row_valid(n: int, c: int, r: int, cap: int, pool_rows: int) -> bool:
    """MTP3 row guard (fused_li_manage_mtp_kernel.h:218-233)."""
    return (n >= TOPK and n <= cap and 0 <= r < pool_rows and c > 0 and c >= min(n, UNION_CAP)
            and c <= MAX_CACHE_TOKENS and c <= n)


def lim_manage_row(scores: np.ndarray, pool_row: np.ndarray, n: int, c: int):
    """One MTP0 request: returns (src[2048], dst[2048], miss_count) and
    updates ``pool_row`` in place."""
    sel = topk_mask(scores[:n], TOPK)
    slots, cached, state, tok, skey = _slot_tables(pool_row, n, c, sel, scores[:n])
    misses = np.nonzero(sel & ~cached)[0]
    m = int(misses.size)
    victims = _victim_slots(c, m, state, skey)
    nv = victims.size
    dst_m = np.full(m, -1, dtype=np.int64)
    dst_m[:nv] = victims
    # pool update: evict victims held by candidate tokens, map misses
    for v in victims:
        if state[v] == 2:
            pool_row[tok[v]] = -1
    pool_row[misses[:nv]] = victims
    hit_slots = np.sort(np.nonzero(state == 1)[0])[::-1]
    src = np.concatenate([misses, tok[hit_slots]]).astype(np.int64)
    dst = np.concatenate([dst_m, hit_slots]).astype(np.int64)
    out_src = np.full(TOPK, -1, dtype=np.int32)
    out_dst = np.full(TOPK, -1, dtype=np.int32)
    k = min(TOPK, src.size)
    out_src[:k] = src[:k]
    out_dst[:k] = dst[:k]
    return out_src, out_dst, m


def fused_li_manage(query, weights, key_cache, block_table, num_candidates, num_cache, pool_entries, pool,
                    topk_src, topk_dst, miss_counts, dtype: str = "bf16", scores=None):
    """Batch MTP0 LIM.  Mutates pool / topk_src / topk_dst / miss_counts.

    query [B,H,128], weights [B,H], key_cache [blocks,128,1,128] as 16-bit
    patterns; integer arrays int32.  ``scores`` (optional list) receives the
    per-request float64 scores.
    """
    q = bits_to_f32(query, dtype)
    w = bits_to_f32(weights, dtype)
    kc = bits_to_f32(key_cache, dtype)
    B = q.shape[0]
    cap = pool.shape[1]
    for b in range(B):
        n, c, r = int(num_candidates[b]), int(num_cache[b]), int(pool_entries[b])
        if not lim_row_valid(n, c, r, cap, pool.shape[0]):
            miss_counts[b] = 0
            if scores is not None:
                scores.append(None)
            continue
        s = index_scores_paged(q[b], w[b], kc, block_table[b], n)
        if scores is not None:
            scores.append(s)
        src, dst, m = lim_manage_row(s, pool[r], n, c)
        topk_src[b, 0] = src
        topk_dst[b, 0] = dst
        miss_counts[b] = m


def ordered_union(rows) -> np.ndarray:
    """Ordered union: first row, then each later row's new tokens
    (ut_ops/test_fused_li_manage_mtp.py:127-137)."""
    seen = set()
    out = []
    for row in rows:
        for t in row:
            t = int(t)
            if t not in seen:
                seen.add(t)
                out.append(t)
    return np.asarray(out, dtype=np.int64)


def lim_manage_mtp_row(scores4, pool_row, n: int, c: int):
    """One MTP3 request. scores4 [4, n]. Returns (rows_src[4,2048],
    rows_dst[4,2048], miss_src[m], miss_dst[m]) and updates pool_row."""
    masks = [topk_mask(scores4[q, :n], TOPK) for q in range(MTP_Q)]
    rows = [np.nonzero(mk)[0] for mk in masks]  # ascending token id
    union = ordered_union(rows)
    in_union = np.zeros(n, dtype=bool)
    in_union[union] = True
    smax = np.max(scores4[:, :n], axis=0)
    slots, cached, state, tok, skey = _slot_tables(pool_row, n, c, in_union, smax)
    pre_cached = cached.copy()
    misses = union[~cached[union]]
    m = int(misses.size)
    victims = _victim_slots(c, m, state, skey)
    nv = victims.size
    miss_dst = np.full(m, -1, dtype=np.int64)
    miss_dst[:nv] = victims
    for v in victims:
        if state[v] == 2:
            pool_row[tok[v]] = -1
    pool_row[misses[:nv]] = victims
    new_slot = np.asarray(pool_row[:n]).astype(np.int64).copy()
    new_slot[misses[nv:]] = -1
    rows_src = np.zeros((MTP_Q, TOPK), dtype=np.int32)
    rows_dst = np.zeros((MTP_Q, TOPK), dtype=np.int32)
    for q in range(MTP_Q):
        toks = rows[q]
        rows_src[q] = np.where(pre_cached[toks], -1, toks)
        rows_dst[q] = new_slot[toks]
    return rows_src, rows_dst, misses.astype(np.int32), miss_dst.astype(np.int32)


def fused_li_manage_mtp(query, weights, key_cache, block_table, num_candidates, num_cache, pool_entries, pool,
                        topk_src, topk_dst, miss_src, miss_dst, miss_counts, dtype: str = "bf16", scores=None):
    """Batch MTP3 LIM (query [4B,H,128]).  Mutates the output buffers."""
    q = bits_to_f32(query, dtype)
    w = bits_to_f32(weights, dtype)
    kc = bits_to_f32(key_cache, dtype)
    B = pool_entries.shape[0]
    cap = pool.shape[1]
    for b in range(B):
        n, c, r = int(num_candidates[b]), int(num_cache[b]), int(pool_entries[b])
        if not lim_mtp_row_valid(n, c, r, cap, pool.shape[0]):
            miss_counts[b] = 0
            if scores is not None:
                scores.append(None)
            continue
        s4 = np.stack([index_scores_paged(q[MTP_Q * b + j], w[MTP_Q * b + j], kc, block_table[b], n)
                       for j in range(MTP_Q)])
        if scores is not None:
            scores.append(s4)
        rs, rd, ms, md = lim_manage_mtp_row(s4, pool[r], n, c)
        topk_src[MTP_Q * b:MTP_Q * b + MTP_Q, 0] = rs
        topk_dst[MTP_Q * b:MTP_Q * b + MTP_Q, 0] = rd
        miss_src[b, :ms.size] = ms
        miss_dst[b, :md.size] = md
        miss_counts[b] = ms.size


# --------------------------------------------------------------------------
# scatter_copy
def resolve_row(token: int, table_row: np.ndarray, num_blocks: int) -> int:
    """Physical row of a logical token through a block-table row, -1 if none."""
    if token < 0:
        return -1
    col = token >> 7
    if col >= table_row.shape[0]:
        return -1
    blk = int(table_row[col])
    if blk < 0 or blk >= num_blocks:
        return -1
    return blk * BLOCK + (token & (BLOCK - 1))


def persist_blocks(hbm_ckv, hbm_kpe, dram_ckv, dram_kpe, hbm_ids, dram_ids) -> None:
    """Prefill -> DRAM persistence (nanovllm/models/glm_mla.py:883-889):
    dram_*[dram_ids[i]] = hbm_*[hbm_ids[i]] for every i, CKV and KPE; a pair
    whose ids name no block of the caches is skipped (the reference would
    index with them; the ABI keeps the device from faulting).  Mutates the
    DRAM arrays ([blocks, 128, ...] of any trailing shape)."""
    for h, d in zip(np.asarray(hbm_ids).tolist(), np.asarray(dram_ids).tolist()):
        if 0 <= h < hbm_ckv.shape[0] and 0 <= d < dram_ckv.shape[0]:
            dram_ckv[d] = hbm_ckv[h]
            dram_kpe[d] = hbm_kpe[h]


def finalize_prefill_pool_row(row, num_full_blocks: int, num_sparse_blocks: int, cache_tokens: int,
                              owner: bool = True, block: int = BLOCK) -> bool:
    """The pool-row part of finalize_prefill_offload (glm_mla.py:857-880): the
    owner resets the row to -1; a short request (num_sparse >= num_full)
    maps token t to slot t for t < num_full*block when the budget is
    nonzero.  Returns True when the blocks must be persisted to DRAM."""
    if owner:
        row[:] = -1
    if num_sparse_blocks >= num_full_blocks:
        if owner and cache_tokens > 0 and num_full_blocks > 0:
            row[:num_full_blocks * block] = np.arange(num_full_blocks * block)
        return False
    return True


def scatter_copy(src_ids, dst_slots, copy_counts, hbm_table, dram_table, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv):
    """Row copy DRAM -> HBM by (src, dst) pairs; caches hold raw 16-bit
    patterns and are mutated in place (test_scatter_copy.py:125-147)."""
    B, cap = src_ids.shape
    hk = hbm_kpe.reshape(-1, KPE)
    hc = hbm_ckv.reshape(-1, CKV)
    dk = dram_kpe.reshape(-1, KPE)
    dc = dram_ckv.reshape(-1, CKV)
    hblocks = min(hbm_kpe.shape[0], hbm_ckv.shape[0])
    dblocks = min(dram_kpe.shape[0], dram_ckv.shape[0])
    for b in range(B):
        count = min(max(int(copy_counts[b]), 0), cap)
        for i in range(count):
            s = int(src_ids[b, i])
            d = int(dst_slots[b, i])
            if s < 0 or d < 0:
                continue
            sr = resolve_row(s, dram_table[b], dblocks)
            dr = resolve_row(d, hbm_table[b], hblocks)
            if sr < 0 or dr < 0:
                continue
            hc[dr] = dc[sr]
            hk[dr] = dk[sr]


# --------------------------------------------------------------------------
# first-decode LIDU initialisation (reference nanovllm/models/dsa_offload_ops.py:251-411)
def linear_index_scores(query: np.ndarray, weights: np.ndarray, keys: np.ndarray) -> np.ndarray:
    """s[t] = sum_h w[h] * (q[h] . k[t]) in float64 -- the initialisation
    score has no ReLU (dsa_offload_ops.py:306-311)."""
    q = np.asarray(query, np.float64).reshape(-1, IDX)
    w = np.asarray(weights, np.float64).reshape(-1)
    return (np.asarray(keys, np.float64) @ q.T) @ w


def _lidu_init_checks(candidate_len: int, cache_tokens: int, block_size: int = BLOCK) -> None:
    """The reference's argument errors (dsa_offload_ops.py:280-294)."""
    if cache_tokens < TOPK:
        raise ValueError(f"LIDU nonzero cache budget must be >= {TOPK}, got {cache_tokens}.")
    if candidate_len < cache_tokens:
        raise ValueError(f"LIDU cache budget {cache_tokens} exceeds source length {candidate_len}.")
    if candidate_len % int(block_size):
        raise ValueError("LIDU source must consist only of complete blocks.")


def initialize_lidu_row(query, weights, key_cache, index_table_row, candidate_len: int, cache_tokens: int,
                        slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_table_row, dram_table_row,
                        dtype: str = "bf16"):
    """Top-C of the linear scores over tokens [0, candidate_len) (ties to the
    lower token), slot i given to the i-th smallest selected token, every
    other entry of the pool row set to -1, and the C rows copied DRAM -> HBM
    (dsa_offload_ops.py:251-360).  The reference assigns slots in the order
    torch.topk(sorted=False) returns the tokens, which is implementation-
    defined; ascending token order is this build's canonical choice.
    Mutates slots_row and the HBM caches; returns (source_ids, slots) or
    None when cache_tokens <= 0."""
    n, c = int(candidate_len), int(cache_tokens)
    if c <= 0:
        return None
    _lidu_init_checks(n, c)
    scores = index_scores_paged(bits_to_f32(query, dtype), bits_to_f32(weights, dtype), bits_to_f32(key_cache, dtype),
                                index_table_row, n, score_fn=linear_index_scores)
    sel = np.nonzero(topk_mask(scores, c))[0].astype(np.int32)
    slots = np.arange(c, dtype=np.int32)
    slots_row[:] = -1
    slots_row[sel] = slots
    scatter_copy(sel[None, :], slots[None, :], np.array([c], np.int32), np.asarray(hbm_table_row)[None],
                 np.asarray(dram_table_row)[None], hbm_kpe, hbm_ckv, dram_kpe, dram_ckv)
    return sel, slots


def initialize_lidu_row_shared(slots_row, cache_tokens: int, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_table_row,
                               dram_table_row):
    """A shared IndexShare layer: copy this layer's DRAM rows of every token
    the owner's pool row caches (ascending token) to its slot
    (dsa_offload_ops.py:363-411).  Returns (source_ids, slots) or None."""
    c = int(cache_tokens)
    if c <= 0:
        return None
    src = np.nonzero(np.asarray(slots_row) >= 0)[0].astype(np.int32)
    dst = np.asarray(slots_row)[src].astype(np.int32)
    if src.size != c:
        raise RuntimeError(f"Shared layer LIDU initialization found {src.size} cached tokens, expected {c}.")
    scatter_copy(src[None, :], dst[None, :], np.array([c], np.int32), np.asarray(hbm_table_row)[None],
                 np.asarray(dram_table_row)[None], hbm_kpe, hbm_ckv, dram_kpe, dram_ckv)
    return src, dst


# --------------------------------------------------------------------------
# sparse-tail attention
def attention_keys(seq_kv: int, c: int, topk_row: np.ndarray, rows_per_request: int, q: int):
    """(slot list, visible length) of one query row, or (None, L) if the row
    outputs zeros (kernel_mla.h:325-353)."""
    L = int(seq_kv)
    if rows_per_request > 1:
        hidden = rows_per_request - 1 - q
        L = L - hidden if L > hidden else 0
    L = max(L, 0)
    if c == 0:
        return np.arange(L, dtype=np.int64), L
    if c >= TOPK and c <= L:
        return np.concatenate([np.asarray(topk_row, np.int64), np.arange(c, L, dtype=np.int64)]), L
    return None, L


def sparse_tail_attention(query_rope, query, seq_kv, num_cache, topk_dst, hbm_table, hbm_kpe, hbm_ckv, scale,
                          rows_per_request: int = 1, dtype: str = "bf16", precision=np.float64):
    """Golden attention -> float array [R, N, 512]."""
    qn = bits_to_f32(query, dtype).astype(precision)
    qr = bits_to_f32(query_rope, dtype).astype(precision)
    kc = bits_to_f32(hbm_ckv, dtype).reshape(-1, CKV)
    kr = bits_to_f32(hbm_kpe, dtype).reshape(-1, KPE)
    hblocks = hbm_ckv.shape[0]
    R, N, _ = qn.shape
    out = np.zeros((R, N, CKV), dtype=precision)
    for row in range(R):
        b = row // rows_per_request
        q = row % rows_per_request
        slots, L = attention_keys(int(seq_kv[b]), int(num_cache[b]), topk_dst[row, 0], rows_per_request, q)
        if slots is None:
            continue
        phys = np.array([resolve_row(int(s), hbm_table[b], hblocks) if 0 <= s < L else -1 for s in slots],
                        dtype=np.int64)
        phys = phys[phys >= 0]
        if phys.size == 0:
            continue
        k = kc[phys].astype(precision)
        kp = kr[phys].astype(precision)
        logits = (qn[row] @ k.T + qr[row] @ kp.T) * precision(scale)
        logits -= logits.max(axis=1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=1, keepdims=True)
        out[row] = p @ k
    return out


def fused_copy_sfa(query_rope, query, seq_kv, num_cache, topk_dst, topk_src, miss_counts, hbm_table, dram_table,
                   hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, scale, dtype: str = "bf16", precision=np.float64):
    """scatter_copy(topk_src[b,:m] -> topk_dst[b,0,:m]) then attention.
    Mutates the HBM caches; returns the attention output."""
    B = topk_src.shape[0]
    scatter_copy(topk_src, topk_dst.reshape(B, -1), miss_counts, hbm_table, dram_table,
                 hbm_kpe.reshape(hbm_kpe.shape[0], BLOCK, KPE), hbm_ckv.reshape(hbm_ckv.shape[0], BLOCK, CKV),
                 dram_kpe, dram_ckv)
    return sparse_tail_attention(query_rope, query, seq_kv, num_cache, topk_dst, hbm_table, hbm_kpe, hbm_ckv,
                                 scale, 1, dtype, precision)


def fused_copy_sfa_mtp(query_rope, query, seq_kv, num_cache, topk_dst, miss_src, miss_dst, miss_counts, hbm_table,
                       dram_table, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, scale, dtype: str = "bf16",
                       precision=np.float64):
    """scatter_copy(union misses) then MTP3 attention."""
    scatter_copy(miss_src, miss_dst, miss_counts, hbm_table, dram_table,
                 hbm_kpe.reshape(hbm_kpe.shape[0], BLOCK, KPE), hbm_ckv.reshape(hbm_ckv.shape[0], BLOCK, CKV),
                 dram_kpe, dram_ckv)
    return sparse_tail_attention(query_rope, query, seq_kv, num_cache, topk_dst, hbm_table, hbm_kpe, hbm_ckv,
                                 scale, MTP_Q, dtype, precision)
