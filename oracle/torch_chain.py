"""Vectorised PyTorch-CPU restatement of the MTP0 chain -- TEST INFRASTRUCTURE ONLY.

The timed CPU baseline of ``bench.py`` (``cpu_baseline``) and nothing else:
only ``tests/`` and that leg of ``bench.py`` import it.  It computes what
``oracle/dsa_oracle.py`` computes -- the reference's golden chain
(ut_ops/test_fused_li_manage.py, ut_ops/test_scatter_copy.py:125-147,
ut_ops/test_sparse_tail_attention.py:190-216), with this build's canonical
victim and row-order rules -- but batched over requests with torch tensor
ops on every host core, the way a CPU implementation of the layer-step
would run:

* ``fused_li_manage``: scores as two batched fp32 products
  (keys x queries, ReLU, x head weights; fused_li_manage_service_cube.h:351,
  fused_li_manage_vector.h:97-167), top-2048 by ``torch.topk`` with ties at
  the threshold taken in ascending token order, hit/miss split against the
  pool rows, victims by one stable sort of the slot keys, and the pool update
  and output rows by scatters (row guards of fused_li_manage_kernel.h:261-290);
* ``fused_copy_sfa``: the miss rows gathered from DRAM and scattered into
  the HBM caches in one indexed copy, then attention over the 2048 selected
  slots plus the tail as two batched fp32 products with a masked softmax
  (kernel_mla.h:325-353).

Scores are fp32 here (float64 in the numpy oracle), so the two select the
same tokens on inputs without near-ties at the selection and victim
boundaries, which is what the workload generator's guard provides;
tests/test_torch_chain.py checks every output against the numpy oracle on
such inputs.  Tensors are CPU torch tensors; 16-bit caches keep their dtype.
"""

from __future__ import annotations

import torch

BLOCK = 128
TOPK = 2048
CKV = 512
KPE = 64
MAX_CACHE_TOKENS = (1 << 14) - 1
MAX_ACTUAL_SEQ_LEN = (1 << 21) - 1
_FMAX = torch.finfo(torch.float32).max


def _rows_valid(n, c, r, cap, pool_rows):
    """MTP0 row guard (fused_li_manage_kernel.h:261-290, plus C <= 16383)."""
    return ((n > 0) & (n <= MAX_ACTUAL_SEQ_LEN) & (n <= cap) & (r >= 0) & (r < pool_rows) & (c >= TOPK)
            & (c <= MAX_CACHE_TOKENS) & (c <= n))


def index_scores(query, weights, key_cache, block_table, n):
    """fp32 scores [B, T] of logical tokens [0, T), T = max(n) rounded to
    blocks; tokens >= n[b] score -inf, tokens of unmapped blocks -FLT_MAX."""
    B = query.shape[0]
    T = int(n.max()) if B else 0
    nb = (T + BLOCK - 1) // BLOCK
    table = block_table[:, :nb].long()
    blocks = key_cache.shape[0]
    bad = (table < 0) | (table >= blocks)
    keys = key_cache.view(blocks, BLOCK, -1)[table.clamp(0, blocks - 1)]  # [B, nb, 128, 128]
    keys = keys.view(B, nb * BLOCK, -1).float()
    dots = torch.bmm(keys, query.float().transpose(1, 2))  # [B, T', H]
    s = torch.bmm(dots.clamp_min_(0.0), weights.float().unsqueeze(2)).squeeze(2)  # [B, T']
    s = torch.where(s == 0, torch.zeros_like(s), s)  # one zero: -0 and +0 rank equal
    s.view(B, nb, BLOCK).masked_fill_(bad.unsqueeze(2), -_FMAX)
    t = torch.arange(nb * BLOCK)
    s.masked_fill_(t.unsqueeze(0) >= n.unsqueeze(1), float("-inf"))
    return s


def fused_li_manage(query, weights, key_cache, block_table, num_candidates, num_cache, pool_entries, pool,
                    topk_src, topk_dst, miss_counts) -> None:
    """Batch MTP0 LIM; mutates pool / topk_src / topk_dst / miss_counts."""
    B = query.shape[0]
    cap = pool.shape[1]
    n = num_candidates.long()
    c = num_cache.long()
    r = pool_entries.long()
    valid = _rows_valid(n, c, r, cap, pool.shape[0])
    miss_counts.copy_(torch.zeros_like(miss_counts))
    if not bool(valid.any()):
        return
    vi = torch.nonzero(valid).squeeze(1)
    n, c, r = n[vi], c[vi], r[vi]
    s = index_scores(query[vi], weights[vi], key_cache, block_table[vi], n)
    Bv, T = s.shape
    tok = torch.arange(T)
    # ---- top-2048, ties at the threshold to the lower token ----------------
    thr = torch.topk(s, TOPK, dim=1).values[:, TOPK - 1:TOPK]
    above = s > thr
    eq = s == thr
    need = TOPK - above.sum(1, keepdim=True)
    sel = above | (eq & (torch.cumsum(eq.int(), 1) <= need))
    # ---- hit / miss against the pool rows ------------------------------------
    P = pool[r][:, :T].long()
    cached = (P >= 0) & (P < c.unsqueeze(1)) & (tok.unsqueeze(0) < n.unsqueeze(1))
    miss = sel & ~cached
    m = miss.sum(1)
    Cmax = int(c.max())
    dump = Cmax  # column that takes the scatters of tokens owning no slot
    idx = torch.where(cached, P, torch.full_like(P, dump))
    state = torch.zeros(Bv, Cmax + 1, dtype=torch.int8)  # 0 free, 1 hit, 2 cached and unselected
    state.scatter_(1, idx, torch.where(sel, 1, 2).to(torch.int8))
    tok_of = torch.full((Bv, Cmax + 1), -1, dtype=torch.long).scatter_(1, idx, tok.expand(Bv, T))
    skey = torch.full((Bv, Cmax + 1), float("-inf")).scatter_(1, idx, s)
    slot = torch.arange(Cmax + 1)
    skey = torch.where(state == 2, skey, torch.full_like(skey, float("-inf")))  # free slots rank first
    nonhit = (state != 1) & (slot.unsqueeze(0) < c.unsqueeze(1))
    skey = torch.where(nonhit, skey, torch.full_like(skey, float("inf")))
    # ---- victims: the m smallest keys (ties to the lower slot), ascending slot
    order = torch.sort(skey, dim=1, stable=True).indices
    nv = torch.minimum(m, nonhit.sum(1))
    rank = torch.arange(Cmax + 1).unsqueeze(0)
    chosen = torch.zeros(Bv, Cmax + 1, dtype=torch.bool).scatter_(1, order, rank < nv.unsqueeze(1))
    big = Cmax + 1 + T
    vslots = torch.sort(torch.where(chosen, slot.unsqueeze(0), big), dim=1).values[:, :TOPK]
    mtok = torch.sort(torch.where(miss, tok.unsqueeze(0), big), dim=1).values[:, :TOPK]
    j = torch.arange(TOPK).unsqueeze(0)
    has_slot = j < nv.unsqueeze(1)
    is_miss = j < m.unsqueeze(1)
    # ---- pool update: victims' tokens lose their slot, misses take them ----
    prow = pool[r].long()
    vtok = tok_of.gather(1, vslots.clamp_max(Cmax))
    evict = has_slot & (vtok >= 0)
    col = torch.where(evict, vtok, torch.full_like(vtok, cap))
    prow_ext = torch.cat([prow, torch.zeros(Bv, 1, dtype=torch.long)], 1)
    prow_ext.scatter_(1, col, torch.full_like(col, -1))
    col = torch.where(has_slot, mtok, torch.full_like(mtok, cap))
    prow_ext.scatter_(1, col, vslots)
    pool[r] = prow_ext[:, :cap].to(pool.dtype)
    # ---- output rows: [misses ascending] ++ [hits by descending old slot] ---
    hit_slots = torch.sort(torch.where(state == 1, slot.unsqueeze(0), -1), dim=1, descending=True).values
    hit_tok = tok_of.gather(1, hit_slots.clamp_min(0))
    pos = (m.unsqueeze(1) + torch.arange(Cmax + 1).unsqueeze(0)).clamp_max(TOPK)  # TOPK = dump column
    src = torch.full((Bv, TOPK + 1), -1, dtype=torch.long)
    dst = torch.full((Bv, TOPK + 1), -1, dtype=torch.long)
    live = hit_slots >= 0
    src.scatter_(1, torch.where(live, pos, TOPK), torch.where(live, hit_tok, -1))
    dst.scatter_(1, torch.where(live, pos, TOPK), torch.where(live, hit_slots, -1))
    src[:, :TOPK] = torch.where(is_miss, mtok, src[:, :TOPK])
    dst[:, :TOPK] = torch.where(is_miss, torch.where(has_slot, vslots, -1), dst[:, :TOPK])
    topk_src[vi] = src[:, :TOPK].to(topk_src.dtype).view(Bv, 1, TOPK)
    topk_dst[vi] = dst[:, :TOPK].to(topk_dst.dtype).view(Bv, 1, TOPK)
    miss_counts[vi] = m.to(miss_counts.dtype)


def _physical_rows(slots, table, blocks):
    """Physical rows of logical slots through block-table rows; -1 if none."""
    col = slots >> 7
    ok = (slots >= 0) & (col < table.shape[1])
    blk = table.gather(1, col.clamp(0, table.shape[1] - 1)).long()
    ok &= (blk >= 0) & (blk < blocks)
    return torch.where(ok, blk * BLOCK + (slots & (BLOCK - 1)), torch.full_like(slots, -1))


def scatter_copy(src_ids, dst_slots, copy_counts, hbm_table, dram_table, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv):
    """DRAM -> HBM rows for pairs i < copy_counts[b] (skip rules of
    kvcache_scatter_copy_kernel.h:141-177); one indexed copy per cache."""
    B, cap = src_ids.shape
    s = src_ids.long()
    d = dst_slots.long()
    live = torch.arange(cap).unsqueeze(0) < copy_counts.long().clamp(0, cap).unsqueeze(1)
    hblocks = min(hbm_kpe.shape[0], hbm_ckv.shape[0])
    dblocks = min(dram_kpe.shape[0], dram_ckv.shape[0])
    sr = _physical_rows(s, dram_table, dblocks)
    dr = _physical_rows(d, hbm_table, hblocks)
    ok = live & (s >= 0) & (d >= 0) & (sr >= 0) & (dr >= 0)
    sr, dr = sr[ok], dr[ok]
    hbm_ckv.view(-1, CKV)[dr] = dram_ckv.reshape(-1, CKV)[sr]
    hbm_kpe.view(-1, KPE)[dr] = dram_kpe.reshape(-1, KPE)[sr]


def sparse_tail_attention(query_rope, query, seq_kv, num_cache, topk_dst, hbm_table, hbm_kpe, hbm_ckv, scale,
                          out) -> None:
    """MTP0 attention over topk_dst ++ [C, L) (kernel_mla.h:325-353): fp32
    products, masked softmax, written to ``out`` in its dtype.  Rows with
    C == 0 attend [0, L); rows outside the rules are zeros."""
    R, H, _ = query.shape
    L = seq_kv.long()
    c = num_cache.long()
    sparse = (c >= TOPK) & (c <= L)
    dense = (c == 0) & (L > 0)
    out.zero_()
    blocks = hbm_ckv.shape[0]
    kc = hbm_ckv.view(-1, CKV)
    kr = hbm_kpe.view(-1, KPE)
    q = torch.cat([query.float(), query_rope.float()], 2)  # [R, H, 576]
    for rows, make in ((torch.nonzero(sparse).squeeze(1), "sparse"), (torch.nonzero(dense).squeeze(1), "dense")):
        if rows.numel() == 0:
            continue
        Lr, cr = L[rows], c[rows]
        if make == "sparse":
            tail = int((Lr - cr).max())
            slots = torch.cat([topk_dst[rows].view(-1, TOPK).long(),
                               cr.unsqueeze(1) + torch.arange(max(tail, 0)).unsqueeze(0)], 1)
            keep = torch.cat([torch.ones(rows.numel(), TOPK, dtype=torch.bool),
                              torch.arange(max(tail, 0)).unsqueeze(0) < (Lr - cr).unsqueeze(1)], 1)
        else:
            K = int(Lr.max())
            slots = torch.arange(K).unsqueeze(0).expand(rows.numel(), K)
            keep = slots < Lr.unsqueeze(1)
        phys = _physical_rows(slots, hbm_table[rows], blocks)
        keep &= (phys >= 0) & (slots < Lr.unsqueeze(1))
        pr = phys.clamp_min(0)
        k = torch.cat([kc[pr].float(), kr[pr].float()], 2)  # [r, K, 576]
        logits = torch.bmm(q[rows], k.transpose(1, 2)) * scale
        logits.masked_fill_(~keep.unsqueeze(1), float("-inf"))
        p = torch.softmax(logits, dim=2)
        p = torch.nan_to_num(p, nan=0.0)  # a row with no usable key
        o = torch.bmm(p, k[:, :, :CKV])
        out[rows] = o.to(out.dtype)


def fused_copy_sfa(query_rope, query, seq_kv, num_cache, topk_dst, topk_src, miss_counts, hbm_table, dram_table,
                   hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, scale, out) -> None:
    """scatter_copy of each row's first miss_counts pairs, then attention."""
    B = topk_src.shape[0]
    scatter_copy(topk_src.view(B, -1), topk_dst.view(B, -1), miss_counts, hbm_table, dram_table, hbm_kpe, hbm_ckv,
                 dram_kpe, dram_ckv)
    sparse_tail_attention(query_rope, query, seq_kv, num_cache, topk_dst, hbm_table, hbm_kpe, hbm_ckv, scale, out)
