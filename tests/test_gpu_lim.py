"""fused_li_manage / fused_li_manage_mtp on the GPU vs the oracle.

* closed-form index (score == token id, ut_ops/test_fused_li_manage.py:146-173)
  with the reference's structured cache state, 32 and 64 index heads, a
  source that crosses the 18-bit boundary (262272 tokens, the reference
  default ``--seq-lens``), the behavioural invariants and the repeated update;
* random margin-guarded workloads: every integer output and the updated pool
  bit-exact against the oracle, bf16 and fp16;
* MTP3 union bookkeeping bit-exact;
* row guards: invalid rows only get miss_counts = 0.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import ints, oracle_lim
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
TOPK = 2048


def _run_lim(dcase, mtp=False):
    from nanovllm_amd import dsa_offload_ops as ops

    t = dcase.tensors
    if mtp:
        ops.fused_li_manage_mtp(t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
                                t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"],
                                t["cache_slots_pool"], t["topk_src_ids"], t["topk_dst_slots"], t["miss_src_ids"],
                                t["miss_dst_slots"], t["miss_counts"])
    else:
        ops.fused_li_manage(t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
                            t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"],
                            t["cache_slots_pool"], t["topk_src_ids"], t["topk_dst_slots"], t["miss_counts"])
    torch.cuda.synchronize()


def _structured_case(heads, batch, seq_len, cache_tokens, miss_count, seed=7):
    """The reference's build_case (test_fused_li_manage.py:127-243)."""
    from nanovllm_amd.workloads import ChainCase

    blocks = (seq_len + 127) // 128
    cap = blocks * 128
    q = torch.zeros(batch, heads, 128)
    q[:, 0, :4] = torch.tensor([1.0, 64.0, 4096.0, 262144.0])
    w = torch.zeros(batch, heads)
    w[:, 0] = 1
    ids = torch.arange(cap)
    key = torch.zeros(batch, blocks, 128, 1, 128)
    key[..., 0, 0] = (ids % 64).view(blocks, 128).float()
    key[..., 0, 1] = ((ids // 64) % 64).view(blocks, 128).float()
    key[..., 0, 2] = ((ids // 4096) % 64).view(blocks, 128).float()
    key[..., 0, 3] = (ids // 262144).view(blocks, 128).float()
    table = torch.arange(batch * blocks, dtype=torch.int32).view(batch, blocks)
    pool_size = batch + 1
    entries = torch.arange(batch, 0, -1, dtype=torch.int32)
    pool = torch.full((pool_size, cap), -1, dtype=torch.int32)
    topk = np.arange(seq_len - TOPK, seq_len)
    hit = topk[miss_count:]
    other_count = cache_tokens - hit.size
    lower = seq_len - TOPK
    others = (np.arange(other_count) * lower) // other_count if other_count else np.zeros(0, np.int64)
    cached = torch.from_numpy(np.concatenate([hit, others]))
    g = torch.Generator().manual_seed(seed)
    for row in range(batch):
        pool[int(entries[row]), cached] = torch.randperm(cache_tokens, generator=g, dtype=torch.int32)
    t = {
        "query_index": q.to(torch.bfloat16), "index_weights": w.to(torch.bfloat16),
        "index_key_cache": key.view(batch * blocks, 128, 1, 128).to(torch.bfloat16), "index_block_table": table,
        "num_candidate_tokens": torch.full((batch,), seq_len, dtype=torch.int32),
        "num_cache_tokens": torch.full((batch,), cache_tokens, dtype=torch.int32), "req_pool_entries": entries,
        "cache_slots_pool": pool, "topk_src_ids": torch.full((batch, 1, TOPK), -1, dtype=torch.int32),
        "topk_dst_slots": torch.full((batch, 1, TOPK), -1, dtype=torch.int32),
        "miss_counts": torch.full((batch,), -1, dtype=torch.int32),
    }
    return ChainCase(t, {})


def _validate(dcase, old_pool, seq_len, cache_tokens, expected_miss):
    """Port of validate_outputs (test_fused_li_manage.py:314-426)."""
    t = dcase.tensors
    B = t["num_candidate_tokens"].numel()
    counts = ints(t["miss_counts"])
    assert counts.tolist() == [expected_miss] * B
    src = ints(t["topk_src_ids"]).reshape(B, TOPK).astype(np.int64)
    dst = ints(t["topk_dst_slots"]).reshape(B, TOPK).astype(np.int64)
    pool = ints(t["cache_slots_pool"])
    entries = ints(t["req_pool_entries"])
    for r in range(pool.shape[0]):
        if r not in set(entries.tolist()):
            assert np.array_equal(pool[r], old_pool[r]), f"unmapped pool row {r} modified"
    for b in range(B):
        s, d = src[b], dst[b]
        assert np.array_equal(np.sort(s), np.arange(seq_len - TOPK, seq_len))
        assert d.min() >= 0 and d.max() < cache_tokens and np.unique(d).size == TOPK
        old = old_pool[entries[b]][s]
        miss = old == -1
        assert miss[:expected_miss].all() and not miss[expected_miss:].any()
        assert np.array_equal(d[expected_miss:], old[expected_miss:])
        assert np.array_equal(pool[entries[b]][s], d)
        valid = pool[entries[b]][pool[entries[b]] >= 0]
        assert valid.size == cache_tokens and np.unique(valid).size == cache_tokens
    return pool


@pytest.mark.parametrize("heads,batch,seq_len,cache_tokens,miss", [
    (32, 2, 20480, 2048, 205),
    (64, 2, 20480, 2048, 205),
    (32, 1, 262272, 6144, 300),
    (64, 3, 65536, 8192, 150),
])
def test_lim_closed_form_and_repeat(heads, batch, seq_len, cache_tokens, miss):
    print(f"LIM closed-form heads={heads} B={batch} N={seq_len} C={cache_tokens} miss={miss}", flush=True)
    case = _structured_case(heads, batch, seq_len, cache_tokens, miss)
    expect = oracle_lim(case)
    old_pool = ints(case["cache_slots_pool"])
    d = case.to_device("cuda")
    _run_lim(d)
    pool1 = _validate(d, old_pool, seq_len, cache_tokens, miss)
    assert np.array_equal(ints(d["topk_src_ids"]), expect["src"])
    assert np.array_equal(ints(d["topk_dst_slots"]), expect["dst"])
    assert np.array_equal(pool1, expect["pool"])
    if seq_len > (1 << 18):
        assert ints(d["topk_src_ids"]).max() >= (1 << 18)
    _run_lim(d)  # same query again: everything is cached now
    _validate(d, pool1, seq_len, cache_tokens, 0)


@pytest.mark.parametrize("n_tokens,cache_tokens", [(12288, 2048), (20480, 6144)])
def test_lim_cold_pool_rows_bit_exact(n_tokens, cache_tokens):
    """Pool rows with nothing cached (every selected token a miss, every
    victim a free slot) beside a warm row: each chunk hands over far more
    misses than its slice holds, so the last chunk re-derives their order;
    every output and the pool bit-exact, and the repeat call has no misses."""
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(3, n_tokens, cache_tokens, [7, 30, 90], seed=29)
    t = case.tensors
    for row in ints(t["req_pool_entries"])[:2]:
        t["cache_slots_pool"][int(row)].fill_(-1)
    print(f"LIM cold pool rows N={n_tokens} C={cache_tokens}", flush=True)
    expect = oracle_lim(case)
    assert (expect["miss_counts"][:2] == 2048).all() and expect["miss_counts"][2] < 2048
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d)
    _assert_matches(d, expect, False)
    _run_lim(d)
    assert (ints(d["miss_counts"]) == 0).all()


def test_lim_large_launch_bit_exact():
    """More chunk workgroups than stay resident beside the last chunk's LDS:
    40 requests on the model runner's 65536-wide tables are 640 chunks, so the
    selection classifies in lim_chunks_kernel and resolves each request in
    lim_resolve_kernel.  Warm and cold pool rows, 4096-16384 tokens, C from
    2048 to 6144: every output and the pool bit-exact (columns past the
    requests untouched), and the repeat call has no misses."""
    from _chain import check_lim, run_lim, widen_layout
    from nanovllm_amd import _lib
    from nanovllm_amd.workloads import make_chain_case

    rng = np.random.default_rng(53)
    B = 40
    lens = [int(x) for x in rng.choice([4096, 6144, 9216, 12288, 16384], size=B)]
    caches = [min(int(x), n) for x, n in zip(rng.choice([2048, 3072, 6144], size=B), lens)]
    case = make_chain_case(B, lens, caches, [int(x) for x in rng.integers(1, 128, size=B)], seed=53)
    t = case.tensors
    for row in ints(t["req_pool_entries"])[:3]:
        t["cache_slots_pool"][int(row)].fill_(-1)
    print("LIM large launch: 40 requests on 65536-wide tables", flush=True)
    expect = oracle_lim(case)
    assert (expect["miss_counts"][:3] == 2048).all()
    d = case.to_device("cuda", host_mapped=False)
    cap0 = d.tensors["cache_slots_pool"].shape[1]
    w = widen_layout(d.tensors, 65536, pad=0)
    wide_init = ints(w["cache_slots_pool"])
    with _lib.KernelTimer(capacity=64) as kt:
        run_lim(w, False)
        torch.cuda.synchronize()
    names = {k for k, _ in kt.records}
    assert {"lim_chunks_kernel", "lim_resolve_kernel"} <= names and "lim_classify_kernel" not in names, names
    check_lim(w, expect, False, "large launch", pool_cols=cap0)
    assert np.array_equal(ints(w["cache_slots_pool"])[:, cap0:], wide_init[:, cap0:])
    run_lim(w, False)
    assert (ints(w["miss_counts"]) == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads", [32, 64])
def test_lim_random_bit_exact(dtype, heads):
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(4, [4096, 6144, 8192, 5120], [2048, 3072, 2560, 2048], [5, 9, 100, 1], index_heads=heads,
                           seed=11 + heads, dtype=dtype)
    print(f"LIM random {dtype} heads={heads} halvings={case.meta['halvings']} miss={case.meta['miss_target']}",
          flush=True)
    expect = oracle_lim(case)
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d)
    assert np.array_equal(ints(d["miss_counts"]), expect["miss_counts"])
    assert np.array_equal(ints(d["topk_src_ids"]), expect["src"])
    assert np.array_equal(ints(d["topk_dst_slots"]), expect["dst"])
    assert np.array_equal(ints(d["cache_slots_pool"]), expect["pool"])
    assert expect["miss_counts"].sum() > 0


@pytest.mark.parametrize("heads", [32, 64])
def test_lim_mtp_bit_exact(heads):
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(3, [9216, 12288, 16384], [8192, 9216, 8320], [4, 10, 60], index_heads=heads, seed=5,
                           mtp=True)
    print(f"LIM MTP heads={heads} halvings={case.meta['halvings']} miss={case.meta['miss_target']}", flush=True)
    expect = oracle_lim(case, mtp=True)
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d, mtp=True)
    mc = ints(d["miss_counts"])
    assert np.array_equal(mc, expect["miss_counts"])
    assert np.array_equal(ints(d["topk_src_ids"]), expect["src"])
    assert np.array_equal(ints(d["topk_dst_slots"]), expect["dst"])
    ms, md = ints(d["miss_src_ids"]), ints(d["miss_dst_slots"])
    for b in range(mc.size):
        assert np.array_equal(ms[b, :mc[b]], expect["miss_src"][b, :mc[b]])
        assert np.array_equal(md[b, :mc[b]], expect["miss_dst"][b, :mc[b]])
    assert np.array_equal(ints(d["cache_slots_pool"]), expect["pool"])


def _tie_case(mtp: bool, positives, seed=11, n_tokens=12288):
    """Scores with exact ties at the top-2048 threshold: query row j of a
    request reads key dim j only, and key dim j is positive for `positives[j]`
    tokens of the request (values 1 + m/128, exact in 16 bits), zero
    otherwise, so after ReLU every other token scores exactly 0 and the
    2048th score is a 0 shared by thousands of tokens (lowest tokens win)."""
    from nanovllm_amd.workloads import make_chain_case

    B, N = 3, n_tokens
    case = make_chain_case(B, N, [8192, 8704, 10240] if mtp else [2048, 4096, 6144], [4, 20, 60], seed=seed,
                           mtp=mtp, guard=False)
    t = case.tensors
    Q = 4 if mtp else 1
    q = torch.zeros(B * Q, 32, 128)
    w = torch.zeros(B * Q, 32)
    for j in range(Q):
        q[j::Q, 0, j] = 1.0
    w[:, 0] = 1.0
    t["query_index"].copy_(q.to(t["query_index"].dtype))
    t["index_weights"].copy_(w.to(t["index_weights"].dtype))
    keys = t["index_key_cache"].view(-1, 128, 128).float()
    keys.zero_()
    table = t["index_block_table"]
    rng = np.random.default_rng(seed)
    for b in range(B):
        for j in range(Q):
            toks = rng.choice(N, size=positives[j], replace=False)
            vals = 1.0 + (rng.integers(0, 128, size=toks.size) / 128.0)
            blk = table[b, torch.from_numpy(toks // 128)].long()
            keys[blk, torch.from_numpy(toks % 128), j] = torch.from_numpy(vals).float()
    t["index_key_cache"].copy_(keys.view_as(t["index_key_cache"]).to(t["index_key_cache"].dtype))
    return case


# MTP0: at 4096 tokens the 3396 tied zeros fit the threshold bin's gather
# list; at 12288 and 40960 they overflow it and the last chunk streams the row.
# MTP3: with fewer than 2048 positive tokens per query row the threshold is
# the 0 shared by thousands of tokens; with more, it falls among the 128
# distinct positive values, each held by ~16-70 tokens, so a few of the ties
# at the threshold are selected and the cutoff falls inside a run of them.
TIE_CASES = [(False, [700], 4096), (False, [700], 12288), (False, [700], 40960),
             (True, [500, 900, 1300, 1900], 12288), (True, [2100, 2600, 3000, 4000], 12288),
             (True, [2100, 3000, 5000, 9000], 40960)]


@pytest.mark.parametrize("mtp,positives,n_tokens", TIE_CASES)
def test_lim_ties_at_threshold_bit_exact(mtp, positives, n_tokens):
    case = _tie_case(mtp, positives, n_tokens=n_tokens)
    print(f"LIM ties mtp={mtp} positives={positives} N={n_tokens}", flush=True)
    expect = oracle_lim(case, mtp=mtp)
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d, mtp=mtp)
    _assert_matches(d, expect, mtp)


def _assert_matches(d, expect, mtp):
    mc = ints(d["miss_counts"])
    assert np.array_equal(mc, expect["miss_counts"])
    assert np.array_equal(ints(d["topk_src_ids"]), expect["src"])
    assert np.array_equal(ints(d["topk_dst_slots"]), expect["dst"])
    if mtp:
        ms, md = ints(d["miss_src_ids"]), ints(d["miss_dst_slots"])
        for b in range(mc.size):
            assert np.array_equal(ms[b, :mc[b]], expect["miss_src"][b, :mc[b]])
            assert np.array_equal(md[b, :mc[b]], expect["miss_dst"][b, :mc[b]])
    assert np.array_equal(ints(d["cache_slots_pool"]), expect["pool"])


@pytest.mark.parametrize("n_tokens", [4096, 12288, 40960])
def test_lim_ties_on_cold_rows_bit_exact(n_tokens):
    """Cold pool rows (nothing cached) with a 2048th score shared by
    thousands of tokens: every selected tied token is an in-bin miss (1348
    per row here), so the last chunk orders a long in-bin miss list (sorted,
    then searched) against the definite misses."""
    case = _tie_case(False, [700], n_tokens=n_tokens)
    t = case.tensors
    for row in ints(t["req_pool_entries"]):
        t["cache_slots_pool"][int(row)].fill_(-1)
    print(f"LIM ties on cold rows N={n_tokens}", flush=True)
    expect = oracle_lim(case)
    valid = np.asarray(case.meta["cache_tokens"]) <= n_tokens  # (C > N disables a row: miss_counts 0)
    assert (expect["miss_counts"][valid] == TOPK).all() and (expect["miss_counts"][~valid] == 0).all()
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d)
    _assert_matches(d, expect, False)


@pytest.mark.parametrize("mtp,positives,n_tokens", TIE_CASES)
def test_lim_unmapped_index_blocks_score_lowest(mtp, positives, n_tokens):
    """Index block-table entries that name no key block (-1, or at or past
    the cache's block count) score -FLT_MAX: below every real score, above
    a free slot when victims are ranked.  The reference reads such an
    entry's memory unchecked (fused_li_manage_service_cube.h:217), so this
    is this library's own guard, restated by the oracle.  One unmapped block
    in the zero-score tie region (block 0), others above it."""
    case = _tie_case(mtp, positives, n_tokens=n_tokens)
    t = case.tensors
    table = t["index_block_table"]
    nblk = t["index_key_cache"].shape[0]
    n = ints(t["num_candidate_tokens"])
    picks = [(0, (int(n[0]) - 1) // 128, -1), (1, int(n[1]) // 256, nblk), (2, int(n[2]) // 192, nblk + 7), (2, 0, -5)]
    for b, col, bad in picks:
        table[b, col] = bad
    print(f"LIM unmapped index blocks mtp={mtp} picks={picks}", flush=True)
    expect = oracle_lim(case, mtp=mtp)
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d, mtp=mtp)
    _assert_matches(d, expect, mtp)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lim_long_rows_small_batch_bit_exact(dtype):
    """Rows of 20480 to 65536 candidates (5 to 16 chunks of 4096 tokens, the
    last chunk of a request to finish resolving the threshold and picking the
    victims) with C = 2048, 6144 and 12288 (the three victim selects: four
    and sixteen slots per thread in registers, streamed); every output and
    the pool bit-exact, and the repeat call has no misses."""
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(4, [40960, 65536, 20480, 49152], [2048, 6144, 12288, 12288], [3, 64, 127, 9], seed=23,
                           dtype=dtype, fast_fill=True)
    print(f"LIM long rows {dtype} halvings={case.meta['halvings']} miss={case.meta['miss_target']}", flush=True)
    expect = oracle_lim(case)
    assert int(expect["miss_counts"].sum()) > 0
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d)
    _assert_matches(d, expect, False)
    _run_lim(d)  # same query again: everything is cached now
    assert (ints(d["miss_counts"]) == 0).all()
    assert np.array_equal(ints(d["cache_slots_pool"]), expect["pool"])


def test_lim_row_guards():
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(5, 4096, 2048, 8, seed=3)
    t = case.tensors
    t["num_candidate_tokens"][0] = 0          # no candidates
    t["num_cache_tokens"][1] = 0              # C == 0
    t["num_cache_tokens"][2] = 1024           # C < 2048
    t["num_cache_tokens"][3] = 8192           # C > candidates
    t["req_pool_entries"][4] = 99             # pool row out of range
    before = ints(t["cache_slots_pool"])
    d = case.to_device("cuda", host_mapped=False)
    _run_lim(d)
    assert ints(d["miss_counts"]).tolist() == [0] * 5
    assert np.array_equal(ints(d["cache_slots_pool"]), before)
    assert np.all(ints(d["topk_src_ids"]) == -1)


def test_lim_mtp_row_guards():
    """MTP3 row guards (fused_li_manage_mtp_kernel.h:218-233, plus C <= 16383,
    the 14-bit slot payload): a disabled request gets miss_counts = 0 and
    nothing else is written -- its four query rows, its miss lists and its
    pool row keep what they held.  Disabled here: N < 2048, C < min(N, 8192),
    C = N = 16384 (above 16383), C > N, a pool row out of range; the last
    request is valid and bit-exact against the oracle."""
    from nanovllm_amd.workloads import make_chain_case

    B = 6
    case = make_chain_case(B, 16384, 8192, 8, seed=4, mtp=True, guard=False)
    t = case.tensors
    t["num_candidate_tokens"][0] = 1024       # N < 2048
    t["num_cache_tokens"][1] = 4096           # C < min(N, 8192)
    t["num_cache_tokens"][2] = 16384          # C = N above the 16383-slot maximum
    t["num_candidate_tokens"][3] = 8064       # C = 8192 > N
    t["req_pool_entries"][4] = 99             # pool row out of range
    expect = oracle_lim(case, mtp=True)
    assert expect["miss_counts"][:5].tolist() == [0] * 5 and expect["miss_counts"][5] > 0
    d = case.to_device("cuda", host_mapped=False)
    dt = d.tensors
    for k in ("topk_src_ids", "topk_dst_slots", "miss_src_ids", "miss_dst_slots", "miss_counts"):
        dt[k].fill_(-5)
    print("LIM MTP3 row guards", flush=True)
    _run_lim(d, mtp=True)
    mc = ints(dt["miss_counts"])
    assert mc.tolist() == expect["miss_counts"].tolist()
    assert np.array_equal(ints(dt["cache_slots_pool"]), expect["pool"])
    src = ints(dt["topk_src_ids"]).reshape(B, 4, -1)
    dst = ints(dt["topk_dst_slots"]).reshape(B, 4, -1)
    assert np.all(src[:5] == -5) and np.all(dst[:5] == -5)
    assert np.array_equal(src[5], expect["src"].reshape(B, 4, -1)[5])
    assert np.array_equal(dst[5], expect["dst"].reshape(B, 4, -1)[5])
    ms, md = ints(dt["miss_src_ids"]), ints(dt["miss_dst_slots"])
    assert np.all(ms[:5] == -5) and np.all(md[:5] == -5)
    assert np.array_equal(ms[5, :mc[5]], expect["miss_src"][5, :mc[5]])
    assert np.array_equal(md[5, :mc[5]], expect["miss_dst"][5, :mc[5]])


def test_lim_meta_and_errors():
    from nanovllm_amd import dsa_offload_ops as ops

    meta = torch.device("meta")
    B = 2
    args = [torch.empty(B, 32, 128, dtype=torch.bfloat16, device=meta), torch.empty(B, 32, dtype=torch.bfloat16,
            device=meta), torch.empty(8, 128, 1, 128, dtype=torch.bfloat16, device=meta),
            torch.empty(B, 4, dtype=torch.int32, device=meta)] + [torch.empty(B, dtype=torch.int32, device=meta)] * 3 + [
            torch.empty(3, 512, dtype=torch.int32, device=meta), torch.empty(B, 1, TOPK, dtype=torch.int32, device=meta),
            torch.empty(B, 1, TOPK, dtype=torch.int32, device=meta), torch.empty(B, dtype=torch.int32, device=meta)]
    assert ops.fused_li_manage(*args) is None
    case = make_bad = None  # noqa: F841
    from nanovllm_amd.workloads import make_chain_case

    d = make_chain_case(1, 4096, 2048, 8, seed=1).to_device("cuda", host_mapped=False)
    t = d.tensors
    with pytest.raises(RuntimeError, match="32 or 64"):
        ops.fused_li_manage(t["query_index"][:, :16].contiguous(), t["index_weights"][:, :16].contiguous(),
                            t["index_key_cache"], t["index_block_table"], t["num_candidate_tokens"],
                            t["num_cache_tokens"], t["req_pool_entries"], t["cache_slots_pool"], t["topk_src_ids"],
                            t["topk_dst_slots"], t["miss_counts"])
    with pytest.raises(RuntimeError, match="state width"):
        ops.fused_li_manage(t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
                            t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"],
                            t["cache_slots_pool"][:, :128].contiguous(), t["topk_src_ids"], t["topk_dst_slots"],
                            t["miss_counts"])
