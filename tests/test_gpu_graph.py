"""The whole layer step captured in a HIP graph and replayed.

The serving path replays the decode step from captured graphs (the
reference's full_decode_graph.py).  Here fused_li_manage(_mtp) ->
fused_copy_sfa(_mtp) is captured once and replayed three times; before each
replay the caller-owned state (pool row, HBM caches, outputs) is put back
with eager torch work on the same stream, and every replay must reproduce
the eager step bit for bit: integer outputs, the updated pool, the HBM
caches after the copy and the attention output (the kernels accumulate in a
fixed order, so repeated runs agree exactly).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, ints

pytestmark = pytest.mark.gpu

STATE = ("cache_slots_pool", "hbm_kv_cache", "hbm_k_rope", "topk_src_ids", "topk_dst_slots", "miss_counts",
         "attention_out")
MTP_STATE = ("miss_src_ids", "miss_dst_slots")


def _step(t, scale, mtp):
    from nanovllm_amd import dsa_offload_ops as ops

    lim = (t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
           t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"], t["cache_slots_pool"],
           t["topk_src_ids"], t["topk_dst_slots"])
    common = (t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
              t["num_cache_tokens"], t["topk_dst_slots"])
    caches = (t["hbm_block_table"], t["dram_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], t["dram_k_rope"],
              t["dram_kv_cache"], scale, t["attention_out"])
    if mtp:
        ops.fused_li_manage_mtp(*lim, t["miss_src_ids"], t["miss_dst_slots"], t["miss_counts"])
        ops.fused_copy_sfa_mtp(*common, t["topk_src_ids"], t["miss_src_ids"], t["miss_dst_slots"],
                               t["miss_counts"], *caches)
    else:
        B = t["query"].shape[0]
        ops.fused_li_manage(*lim, t["miss_counts"])
        ops.fused_copy_sfa(*common, t["topk_src_ids"].view(B, -1), t["miss_counts"], *caches)


def _snapshot(t, names):
    return {k: (bits(t[k]) if t[k].dtype in (torch.bfloat16, torch.float16) else ints(t[k])).copy() for k in names}


@pytest.mark.parametrize("mtp", [False, True])
def test_layer_step_graph_replays_match_eager(mtp):
    from nanovllm_amd.workloads import make_chain_case

    if mtp:
        case = make_chain_case(2, [9216, 12288], [8192, 9216], [4, 33], seed=21, mtp=True)
    else:
        case = make_chain_case(3, [8192, 12288, 16384], [2048, 4096, 2048], [5, 60, 127], seed=21)
    print(f"GRAPH mtp={mtp}", flush=True)
    d = case.to_device("cuda")
    t = d.tensors
    names = STATE + (MTP_STATE if mtp else ())
    initial = {k: t[k].clone() for k in names}
    scale = case.meta["scale"]

    def restore():  # eager work on the current stream between replays
        for k in names:
            t[k].copy_(initial[k])

    _step(t, scale, mtp)  # eager reference (also sizes the op workspaces)
    torch.cuda.synchronize()
    expect = _snapshot(t, names)
    assert int(ints(t["miss_counts"]).sum()) > 0, "the step must copy rows"

    restore()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _step(t, scale, mtp)  # warm the capture stream
    stream.synchronize()
    restore()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _step(t, scale, mtp)
    torch.cuda.synchronize()
    for rep in range(3):
        restore()
        junk = torch.randn(1 << 16, device="cuda").sum()  # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        got = _snapshot(t, names)
        for k in names:
            assert np.array_equal(got[k], expect[k]), (mtp, rep, k)
        del junk
