"""nvdsa_fused_li_manage_noalloc (the allocation-free LIM entry point) through
the C ABI against nvdsa_fused_li_manage with a caller workspace.

Two calls in a row on the static scratch memory, the second with a smaller
input, each on a copy of the same persistent state as a call of the
workspace entry point: every output and the updated pool bit-exact.  The
first call has requests on both manage paths (<= 32768 candidates in
registers, longer ones streamed) and cache budgets whose slot tables live in
the scratch memory; the second reuses the scratch memory the first left
behind.  A batch whose scratch would exceed the static size is rejected
before anything is launched.

Under HIP-graph capture: the call captured, then replayed on two different
inputs written into the captured tensors, each replay bit-exact with the
workspace entry point on the same inputs; and, in a fresh process, the same
with the first call of that process (the one that looks the scratch address
up) made while capturing.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _helpers import ints, oracle_lim

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 32 << 20  # NVDSA_NOALLOC_SCRATCH_BYTES
ARGS = ("query_index", "index_weights", "index_key_cache", "index_block_table", "num_candidate_tokens",
        "num_cache_tokens", "req_pool_entries", "cache_slots_pool", "topk_src_ids", "topk_dst_slots", "miss_counts")
OUTS = ("cache_slots_pool", "topk_src_ids", "topk_dst_slots", "miss_counts")


def _call(t, noalloc: bool) -> int:
    from nanovllm_amd import _lib

    descs = [_lib.describe(t[k]) for k in ARGS]
    refs = [ctypes.byref(d) for d in descs]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        return _lib.lib.nvdsa_fused_li_manage_noalloc(*refs, stream)
    nbytes = _lib.lib.nvdsa_fused_li_manage_workspace_size(t["query_index"].shape[0],
                                                           t["index_block_table"].shape[1] * 128,
                                                           t["query_index"].shape[1])
    ws = torch.empty(nbytes, dtype=torch.uint8, device=t["query_index"].device)
    rc = _lib.lib.nvdsa_fused_li_manage(*refs, ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    return rc


def _compare(case, label, with_oracle=False):
    from nanovllm_amd import _lib

    d = case.to_device("cuda").tensors
    a = dict(d)
    b = dict(d)
    for k in OUTS:
        a[k] = d[k].clone()
        b[k] = d[k].clone()
    b["topk_src_ids"].fill_(-5)
    b["topk_dst_slots"].fill_(-5)
    b["miss_counts"].fill_(-5)
    print(f"NOALLOC {label}: workspace entry point", flush=True)
    assert _call(a, False) == 0, _lib.last_error()
    print(f"NOALLOC {label}: allocation-free entry point", flush=True)
    assert _call(b, True) == 0, _lib.last_error()
    torch.cuda.synchronize()
    for k in OUTS:
        assert np.array_equal(ints(a[k]), ints(b[k])), (label, k)
    assert int(ints(b["miss_counts"]).sum()) > 0, label
    if with_oracle:
        exp = oracle_lim(case)
        assert np.array_equal(ints(b["topk_src_ids"]), exp["src"]), label
        assert np.array_equal(ints(b["cache_slots_pool"]), exp["pool"]), label


def test_noalloc_matches_workspace_entry_point_twice():
    from nanovllm_amd.workloads import make_chain_case

    big = make_chain_case(6, [65536, 32768, 20480, 40960, 8192, 16384], [2048, 8192, 4096, 12288, 2048, 6144],
                          [5, 100, 1, 64, 127, 30], seed=71, fast_fill=True)
    small = make_chain_case(2, [8192, 4096], [2048, 2048], [3, 9], seed=72)
    _compare(big, "call 1 (6 requests, S_cap 65536)")
    _compare(small, "call 2 (2 requests, S_cap 8192)", with_oracle=True)


INPUTS = ("query_index", "index_weights", "index_key_cache", "index_block_table", "num_candidate_tokens",
          "num_cache_tokens", "req_pool_entries", "cache_slots_pool")


def _poison(t) -> None:
    for k in ("topk_src_ids", "topk_dst_slots", "miss_counts"):
        t[k].fill_(-5)


def capture_check(label: str) -> None:
    """Capture nvdsa_fused_li_manage_noalloc in a graph, replay it on two
    inputs and compare each replay with the workspace entry point."""
    from nanovllm_amd import _lib
    from nanovllm_amd.workloads import make_chain_case

    lens, caches, tails = [8192, 20480, 4096], [2048, 4096, 2048], [3, 9, 1]
    cases = [make_chain_case(3, lens, caches, tails, seed=s) for s in (73, 74)]
    g = cases[0].to_device("cuda").tensors
    _poison(g)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print(f"NOALLOC {label}: capture", flush=True)
    with torch.cuda.graph(graph):
        assert _call(g, True) == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert (ints(g["miss_counts"]) == -5).all(), "capture ran the call"
    for i, case in enumerate(cases):
        ref = case.to_device("cuda").tensors
        assert _call(ref, False) == 0, _lib.last_error()
        for k in INPUTS:
            g[k].copy_(case.tensors[k].to("cuda"))
        _poison(g)
        torch.cuda.synchronize()
        print(f"NOALLOC {label}: replay {i}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for k in OUTS:
            assert np.array_equal(ints(g[k]), ints(ref[k])), (label, i, k)
        assert int(ints(g["miss_counts"]).sum()) > 0, (label, i)
    del graph


def test_noalloc_captured_in_a_graph():
    capture_check("graph")


def test_noalloc_first_call_under_capture_in_a_fresh_process():
    """The scratch address is looked up on a device's first call; here that
    call is made while capturing (a fresh process: no earlier call)."""
    import subprocess
    import sys
    from pathlib import Path

    here = Path(__file__).resolve().parent
    code = (f"import sys; sys.path[:0] = [{str(here)!r}, {str(here.parent / 'nanovllm-dsa-offload_amd')!r}, "
            f"{str(here.parent)!r}]\n"
            "import test_zz_no_alloc as T\n"
            "T.capture_check('first call under capture')\n"
            "print('FIRST CALL UNDER CAPTURE OK', flush=True)\n")
    print("NOALLOC fresh process: start", flush=True)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    print(out.stdout[-2000:], out.stderr[-2000:], flush=True)
    assert out.returncode == 0 and "FIRST CALL UNDER CAPTURE OK" in out.stdout


def test_noalloc_rejects_scratch_beyond_its_size():
    from nanovllm_amd import _lib

    B, cols = 64, 1024  # 64 x 131072 fp32 scores alone exceed 32 MiB
    dev = torch.device("cuda")
    need = _lib.lib.nvdsa_fused_li_manage_workspace_size(B, cols * 128, 32)
    assert need > NOALLOC_BYTES
    i32 = dict(dtype=torch.int32, device=dev)
    t = {
        "query_index": torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=dev),
        "index_weights": torch.zeros(B, 32, dtype=torch.bfloat16, device=dev),
        "index_key_cache": torch.zeros(1, 128, 1, 128, dtype=torch.bfloat16, device=dev),
        "index_block_table": torch.zeros(B, cols, **i32),
        "num_candidate_tokens": torch.full((B,), 4096, **i32),
        "num_cache_tokens": torch.full((B,), 2048, **i32),
        "req_pool_entries": torch.arange(B, **i32),
        "cache_slots_pool": torch.full((B, cols * 128), -1, **i32),
        "topk_src_ids": torch.full((B, 1, 2048), -9, **i32),
        "topk_dst_slots": torch.full((B, 1, 2048), -9, **i32),
        "miss_counts": torch.full((B,), -9, **i32),
    }
    print("NOALLOC oversized request", flush=True)
    rc = _call(t, True)
    torch.cuda.synchronize()
    assert rc == 5, rc  # NVDSA_ERR_WORKSPACE
    msg = _lib.last_error()
    assert "fused_li_manage_noalloc" in msg and str(NOALLOC_BYTES) in msg, msg
    assert (ints(t["miss_counts"]) == -9).all()  # nothing ran
