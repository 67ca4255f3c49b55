"""sparse_tail_attention(_mtp) and fused_copy_sfa(_mtp) on the GPU.

* the reference's (C, tail) cases (ut_ops/test_sparse_tail_attention.py:99-108)
  against the float64 golden, for several head counts;
* MTP3 per-query causal visible lengths (test_sparse_tail_attention_mtp.py:314-327);
* fused copy + attention against the composition scatter_copy -> attention:
  HBM caches bit-exact, attention within tolerance, destinations poisoned so
  stale HBM fails (test_fused_copy_sfa.py:421-450), a C=0 row and a
  zero-miss row (:532-602), and against the serial pair run on the GPU.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _helpers import assert_attention_close, bits, dname, ints
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
TOPK = 2048


def _sfa_case(cases, heads, seed, rows_per_request=1, dtype=torch.bfloat16, scale_q=0.25):
    g = torch.Generator().manual_seed(seed)
    B = len(cases)
    lens = [c + t for c, t in cases]
    cols = max(1, math.ceil(max(lens) / 128))
    total = B * cols
    table = torch.randperm(total, generator=g).to(torch.int32).view(B, cols)
    R = B * rows_per_request
    t = {
        "query": (torch.randn(R, heads, 512, generator=g) * scale_q).to(dtype),
        "query_rope": (torch.randn(R, heads, 64, generator=g) * scale_q).to(dtype),
        "hbm_kv_cache": (torch.randn(total, 128, 1, 512, generator=g) * 0.25).to(dtype),
        "hbm_k_rope": (torch.randn(total, 128, 1, 64, generator=g) * 0.25).to(dtype),
        "hbm_block_table": table,
        "num_cache_tokens": torch.tensor([c for c, _ in cases], dtype=torch.int32),
        "actual_seq_lengths_kv": torch.tensor(lens, dtype=torch.int32),
        "actual_seq_lengths_query": torch.arange(rows_per_request, R + 1, rows_per_request, dtype=torch.int32),
        "topk_dst_slots": torch.zeros(R, 1, TOPK, dtype=torch.int32),
    }
    for r in range(R):
        c = cases[r // rows_per_request][0]
        if c >= TOPK:
            t["topk_dst_slots"][r, 0] = torch.randperm(c, generator=g)[:TOPK].to(torch.int32)
    return t


def _golden(t, scale, rows_per_request, dtype):
    return O.sparse_tail_attention(bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]),
                                   ints(t["num_cache_tokens"]), ints(t["topk_dst_slots"]), ints(t["hbm_block_table"]),
                                   bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"]), scale, rows_per_request,
                                   dname(dtype))


def _run_sfa(t, scale, mtp=False):
    from nanovllm_amd import dsa_offload_ops as ops

    d = {k: v.cuda() for k, v in t.items()}
    out = torch.full_like(d["query"], 7.0)
    fn = ops.sparse_tail_attention_mtp if mtp else ops.sparse_tail_attention
    fn(d["query_rope"], d["query"], d["actual_seq_lengths_query"], d["actual_seq_lengths_kv"], d["num_cache_tokens"],
       d["topk_dst_slots"], d["hbm_block_table"], d["hbm_k_rope"], d["hbm_kv_cache"], scale, out)
    torch.cuda.synchronize()
    return out


REF_CASES = [(0, 1), (0, 129), (0, 2049), (2048, 0), (6144, 257), (5120, 1025)]


@pytest.mark.parametrize("heads", [64, 4, 16, 128])
def test_sparse_tail_attention_reference_cases(heads):
    scale = 1.0 / math.sqrt(576)
    t = _sfa_case(REF_CASES, heads, seed=7)
    out = _run_sfa(t, scale)
    gold = _golden(t, scale, 1, torch.bfloat16)
    assert_attention_close(out, gold, label=f"sfa heads={heads}")


def test_sparse_tail_attention_fp16_and_model_scale():
    scale = 192 ** -0.5  # nanovllm/models/glm_mla.py:448
    t = _sfa_case([(2048, 64), (0, 300), (4096, 1)], 64, seed=9, dtype=torch.float16)
    out = _run_sfa(t, scale)
    assert_attention_close(out, _golden(t, scale, 1, torch.float16), torch.float16, label="sfa fp16")


def test_sparse_tail_attention_inactive_rows_are_zero():
    scale = 0.05
    t = _sfa_case([(1024, 10), (2048, 0), (3000, 5)], 64, seed=2)
    t["actual_seq_lengths_kv"][1] = 2047  # C > L
    out = _run_sfa(t, scale)
    assert torch.all(out[0] == 0) and torch.all(out[1] == 0)
    assert_attention_close(out, _golden(t, scale, 1, torch.bfloat16), label="sfa inactive")


@pytest.mark.parametrize("heads", [64, 16])
def test_sparse_tail_attention_mtp(heads):
    scale = 1.0 / math.sqrt(576)
    t = _sfa_case([(2048, 4), (6144, 257), (0, 300), (2048, 3)], heads, seed=13, rows_per_request=4)
    out = _run_sfa(t, scale, mtp=True)
    assert_attention_close(out, _golden(t, scale, 4, torch.bfloat16), label=f"sfa-mtp heads={heads}")


# --------------------------------------------------------------------------
# fused copy + attention
def _chain_after_lim(case, mtp=False):
    """Device case whose LIM outputs come from the oracle (bit-exact with the
    GPU LIM, which test_gpu_lim checks) so the fused op is tested alone."""
    from _helpers import oracle_lim

    exp = oracle_lim(case, mtp=mtp)
    t = case.tensors
    t["topk_src_ids"] = torch.from_numpy(exp["src"])
    t["topk_dst_slots"] = torch.from_numpy(exp["dst"])
    t["miss_counts"] = torch.from_numpy(exp["miss_counts"])
    t["cache_slots_pool"] = torch.from_numpy(exp["pool"])
    if mtp:
        t["miss_src_ids"] = torch.from_numpy(exp["miss_src"])
        t["miss_dst_slots"] = torch.from_numpy(exp["miss_dst"])
    return case


def _oracle_fused(case, mtp=False):
    t = case.tensors
    dt = dname(t["query"].dtype)
    hkpe, hckv = bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"])
    common = dict(dtype=dt)
    if mtp:
        out = O.fused_copy_sfa_mtp(bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]),
                                   ints(t["num_cache_tokens"]), ints(t["topk_dst_slots"]), ints(t["miss_src_ids"]),
                                   ints(t["miss_dst_slots"]), ints(t["miss_counts"]), ints(t["hbm_block_table"]),
                                   ints(t["dram_block_table"]), hkpe, hckv, bits(t["dram_k_rope"]),
                                   bits(t["dram_kv_cache"]), case.meta["scale"], **common)
    else:
        B = t["query"].shape[0]
        out = O.fused_copy_sfa(bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]),
                               ints(t["num_cache_tokens"]), ints(t["topk_dst_slots"]),
                               ints(t["topk_src_ids"]).reshape(B, TOPK), ints(t["miss_counts"]),
                               ints(t["hbm_block_table"]), ints(t["dram_block_table"]), hkpe, hckv,
                               bits(t["dram_k_rope"]), bits(t["dram_kv_cache"]), case.meta["scale"], **common)
    return out, hkpe, hckv


def _run_fused(d, scale, mtp=False):
    from nanovllm_amd import dsa_offload_ops as ops

    t = d.tensors
    out = t["attention_out"]
    out.fill_(7.0)
    if mtp:
        ops.fused_copy_sfa_mtp(t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
                               t["num_cache_tokens"], t["topk_dst_slots"], t["topk_src_ids"], t["miss_src_ids"],
                               t["miss_dst_slots"], t["miss_counts"], t["hbm_block_table"], t["dram_block_table"],
                               t["hbm_k_rope"], t["hbm_kv_cache"], t["dram_k_rope"], t["dram_kv_cache"], scale, out)
    else:
        B = t["query"].shape[0]
        ops.fused_copy_sfa(t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
                           t["num_cache_tokens"], t["topk_dst_slots"], t["topk_src_ids"].view(B, TOPK),
                           t["miss_counts"], t["hbm_block_table"], t["dram_block_table"], t["hbm_k_rope"],
                           t["hbm_kv_cache"], t["dram_k_rope"], t["dram_kv_cache"], scale, out)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_copy_sfa_matches_composition(dtype):
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(4, [4096, 6144, 8192, 4096], [2048, 3072, 2560, 2048], [37, 1, 127, 64], seed=21,
                           dtype=dtype)
    case = _chain_after_lim(case)
    case.tensors["miss_counts"][3] = 0  # a zero-miss row
    print(f"FUSED miss={case['miss_counts'].tolist()}", flush=True)
    gold, hkpe, hckv = _oracle_fused(case)
    d = case.to_device("cuda")
    out = _run_fused(d, case.meta["scale"])
    assert np.array_equal(bits(d["hbm_kv_cache"]), hckv)
    assert np.array_equal(bits(d["hbm_k_rope"]), hkpe)
    assert_attention_close(out, gold, dtype, label=f"fused {dtype}")


def test_fused_copy_sfa_c0_row_and_serial_pair():
    from nanovllm_amd import dsa_offload_ops as ops
    from nanovllm_amd.workloads import make_chain_case

    case = make_chain_case(3, [4096, 4096, 6144], [2048, 0, 2048], [5, 300, 17], seed=4)
    case = _chain_after_lim(case)
    gold, hkpe, hckv = _oracle_fused(case)
    d = case.to_device("cuda")
    d2 = case.to_device("cuda")
    out = _run_fused(d, case.meta["scale"])
    assert np.array_equal(bits(d["hbm_kv_cache"]), hckv)
    assert_attention_close(out, gold, label="fused C=0 row")
    # serial pair on the GPU: scatter_copy then sparse_tail_attention
    t = d2.tensors
    B = 3
    ops.scatter_copy(t["topk_src_ids"].view(B, TOPK), t["topk_dst_slots"].view(B, TOPK), t["miss_counts"],
                     t["hbm_block_table"], t["dram_block_table"], t["hbm_k_rope"].view(-1, 128, 64),
                     t["hbm_kv_cache"].view(-1, 128, 512), t["dram_k_rope"], t["dram_kv_cache"])
    out2 = torch.zeros_like(out)
    ops.sparse_tail_attention(t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
                              t["num_cache_tokens"], t["topk_dst_slots"], t["hbm_block_table"], t["hbm_k_rope"],
                              t["hbm_kv_cache"], case.meta["scale"], out2)
    torch.cuda.synchronize()
    assert torch.equal(d["hbm_kv_cache"].cpu(), d2["hbm_kv_cache"].cpu())
    torch.testing.assert_close(out.float(), out2.float(), rtol=0.02, atol=0.01)


# One request: 4 query rows, 48 + 64 splits over the two attention launches,
# merged by seven 16-split groups of the combine; two requests: 56 splits.
@pytest.mark.parametrize("batch", [2, 1])
def test_fused_copy_sfa_mtp_matches_composition(batch):
    from nanovllm_amd.workloads import make_chain_case

    if batch == 2:
        case = make_chain_case(2, [9216, 12288], [8192, 9216], [4, 33], seed=8, mtp=True)
    else:
        case = make_chain_case(1, [12288], [8192], [33], seed=9, mtp=True)
    case = _chain_after_lim(case, mtp=True)
    gold, hkpe, hckv = _oracle_fused(case, mtp=True)
    d = case.to_device("cuda")
    out = _run_fused(d, case.meta["scale"], mtp=True)
    assert np.array_equal(bits(d["hbm_kv_cache"]), hckv)
    assert np.array_equal(bits(d["hbm_k_rope"]), hkpe)
    assert_attention_close(out, gold, label="fused-mtp")


def test_fused_copy_sfa_mtp_roles_on_separate_xcds():
    """The MTP3 overlap kernel gives workgroups the copy or the attention role
    by linear id, assuming workgroups are dealt to the 8 XCDs round-robin (the
    single-partition mode), so that the copy's host reads and the attention's
    HBM reads never share an XCD (the results do not depend on it, the speed
    does).  Each workgroup records the XCD it ran on (hardware XCC_ID); the
    copy role must cover 5 XCDs and the attention the other 3."""
    from nanovllm_amd import _lib
    from nanovllm_amd.workloads import make_chain_case

    if torch.cuda.get_device_properties(0).multi_processor_count < 256:
        pytest.skip("a partitioned device: fewer than 8 XCDs per device")
    case = _chain_after_lim(make_chain_case(2, [4096, 6144], [2048, 2048], [4, 33], seed=3, mtp=True), mtp=True)
    d = case.to_device("cuda")
    _lib.xcd_roles(reset=True)
    _run_fused(d, case.meta["scale"], mtp=True)  # recording off: no record
    assert _lib.xcd_roles(reset=True) == (0, 0)
    with _lib.record_xcd_roles():
        _run_fused(d, case.meta["scale"], mtp=True)
    copy_xcds, attn_xcds = _lib.xcd_roles(reset=True)
    print(f"copy XCDs {copy_xcds:#04x}, attention XCDs {attn_xcds:#04x}", flush=True)
    assert copy_xcds & attn_xcds == 0, (hex(copy_xcds), hex(attn_xcds))
    assert bin(copy_xcds).count("1") == 5 and bin(attn_xcds).count("1") == 3, (hex(copy_xcds), hex(attn_xcds))
    assert _lib.xcd_roles() == (0, 0)  # the read above cleared the record
