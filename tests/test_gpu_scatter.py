"""scatter_copy on the GPU vs the oracle's apply_reference restatement.

Mirrors ut_ops/test_scatter_copy.py: random block tables, capacities 2048
and 8192, counts from 0 to the full capacity, zero-count no-op, and adds the
skip rules (negative ids, ids beyond a table, -1 table entries) and a count
above the capacity.  DRAM lives in host-mapped memory.  Bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, ints
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _case(seed, batch, source_len, hbm_tokens, cap, counts, dtype=torch.bfloat16):
    from nanovllm_amd.host_memory import host_mapped_pair

    g = torch.Generator().manual_seed(seed)
    sblk = (source_len + 127) // 128
    hblk = (hbm_tokens + 127) // 128
    dram_table = torch.randperm(batch * sblk, generator=g).to(torch.int32).view(batch, sblk)
    hbm_table = torch.randperm(batch * hblk, generator=g).to(torch.int32).view(batch, hblk)
    dram_ckv = torch.randn(batch * sblk, 128, 512, generator=g).to(dtype)
    dram_kpe = torch.randn(batch * sblk, 128, 64, generator=g).to(dtype)
    hbm_ckv = torch.full((batch * hblk, 128, 512), 37.0).to(dtype)  # poisoned destinations
    hbm_kpe = torch.full((batch * hblk, 128, 64), -29.0).to(dtype)
    src = torch.full((batch, cap), -1, dtype=torch.int32)
    dst = torch.full((batch, cap), -1, dtype=torch.int32)
    for b, c in enumerate(counts):
        c = min(c, cap)
        if c:
            src[b, :c] = torch.randperm(source_len, generator=g)[:c].to(torch.int32)
            dst[b, :c] = torch.randperm(hbm_tokens, generator=g)[:c].to(torch.int32)
    dev = torch.device("cuda")
    d_ckv, h_ckv = host_mapped_pair(dram_ckv.shape, dtype, dev)
    d_kpe, h_kpe = host_mapped_pair(dram_kpe.shape, dtype, dev)
    h_ckv.copy_(dram_ckv)
    h_kpe.copy_(dram_kpe)
    return dict(src=src, dst=dst, counts=torch.tensor(counts, dtype=torch.int32), hbm_table=hbm_table,
                dram_table=dram_table, hbm_kpe=hbm_kpe, hbm_ckv=hbm_ckv, dram_kpe=dram_kpe, dram_ckv=dram_ckv,
                d_ckv=d_ckv, d_kpe=d_kpe)


def _run_and_compare(c, label):
    from nanovllm_amd import dsa_offload_ops as ops

    dev = torch.device("cuda")
    g_kpe = c["hbm_kpe"].to(dev)
    g_ckv = c["hbm_ckv"].to(dev)
    print(f"SCATTER case={label}", flush=True)
    ops.scatter_copy(c["src"].to(dev), c["dst"].to(dev), c["counts"].to(dev), c["hbm_table"].to(dev),
                     c["dram_table"].to(dev), g_kpe, g_ckv, c["d_kpe"], c["d_ckv"])
    torch.cuda.synchronize()
    e_kpe, e_ckv = bits(c["hbm_kpe"]), bits(c["hbm_ckv"])
    O.scatter_copy(ints(c["src"]), ints(c["dst"]), ints(c["counts"]), ints(c["hbm_table"]), ints(c["dram_table"]),
                   e_kpe, e_ckv, bits(c["dram_kpe"]), bits(c["dram_ckv"]))
    assert np.array_equal(bits(g_ckv), e_ckv), label
    assert np.array_equal(bits(g_kpe), e_kpe), label
    return g_kpe, g_ckv


@pytest.mark.parametrize("cap,counts", [(2048, [0, 1, 300, 2048]), (8192, [8192, 17, 0, 4000])])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_scatter_copy_bit_exact(cap, counts, dtype):
    c = _case(7, len(counts), 20992, 8320, cap, counts, dtype)
    _run_and_compare(c, f"cap={cap} counts={counts} {dtype}")


def test_scatter_copy_zero_count_is_noop():
    c = _case(3, 2, 4096, 2048, 2048, [0, 0])
    g_kpe, g_ckv = _run_and_compare(c, "zero")
    assert torch.equal(g_ckv.cpu(), c["hbm_ckv"]) and torch.equal(g_kpe.cpu(), c["hbm_kpe"])


def test_scatter_copy_skip_rules_and_count_clamp():
    c = _case(5, 3, 4096, 2048, 64, [64, 10, 10])
    c["src"][0, 3] = -5          # negative source id
    c["dst"][0, 4] = -1          # negative slot
    c["dst"][1, 2] = 2048 + 7    # slot beyond the HBM table
    c["src"][1, 3] = 4096 + 130  # source beyond the DRAM table
    c["dram_table"][2, 1] = -1   # unmapped DRAM block
    c["src"][2, :10] = torch.arange(128, 138, dtype=torch.int32)
    c["counts"][1] = 1000        # above capacity: clamped to 64 (entries past 10 are -1)
    _run_and_compare(c, "skip-rules")


def test_scatter_copy_rejects_bad_shapes():
    from nanovllm_amd import dsa_offload_ops as ops

    c = _case(1, 1, 1024, 1024, 16, [4])
    dev = torch.device("cuda")
    with pytest.raises(RuntimeError, match="HBM CKV"):
        ops.scatter_copy(c["src"].to(dev), c["dst"].to(dev), c["counts"].to(dev), c["hbm_table"].to(dev),
                         c["dram_table"].to(dev), c["hbm_kpe"].to(dev), c["hbm_ckv"][:, :, :256].contiguous().to(dev),
                         c["d_kpe"], c["d_ckv"])
    with pytest.raises(RuntimeError, match="int32"):
        ops.scatter_copy(c["src"].to(dev).long(), c["dst"].to(dev), c["counts"].to(dev), c["hbm_table"].to(dev),
                         c["dram_table"].to(dev), c["hbm_kpe"].to(dev), c["hbm_ckv"].to(dev), c["d_kpe"], c["d_ckv"])
