"""Golden vectors of the chain (tests/golden/chain_golden.npz, written by
tests/golden/make_golden.py from seeded workloads).

* CPU: the oracle reproduces every stored output exactly (its canonical
  results are frozen: a change of the oracle or of the generator fails here).
* GPU: the HIP chain (fused_li_manage(_mtp) -> fused_copy_sfa(_mtp)) matches
  the stored outputs -- ids, slots, miss lists and the updated pool
  bit-exact, the HBM caches after the copy by SHA-256 digest, attention
  within the stated tolerance -- without running the oracle.
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from _helpers import assert_attention_close, bits, ints

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)

_DATA = np.load(GOLDEN / "chain_golden.npz")
NAMES = sorted({k.split("/")[0] for k in _DATA.files})
INT_KEYS = ("src", "dst", "miss_counts", "pool", "miss_src", "miss_dst")


def _fixture(name: str) -> dict:
    out = {}
    for key in _DATA.files:
        case, field = key.split("/", 1)
        if case != name:
            continue
        arr = _DATA[key]
        out[field] = arr.tobytes().decode() if field in ("params", "hbm_kv_digest", "hbm_kpe_digest") else arr
    out["params"] = json.loads(out["params"])
    return out


def test_golden_file_lists_every_case():
    assert NAMES == sorted(make_golden.CASES)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    fx = _fixture(name)
    res = make_golden.run_oracle(make_golden.build_case(fx["params"]), fx["params"]["mtp"])
    for key in INT_KEYS:
        if key in fx:
            assert np.array_equal(res[key], fx[key]), (name, key)
    assert np.array_equal(res["attention"], fx["attention"]), name
    assert res["hbm_kv_digest"] == fx["hbm_kv_digest"] and res["hbm_kpe_digest"] == fx["hbm_kpe_digest"], name


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_chain_matches_golden(name):
    from nanovllm_amd import dsa_offload_ops as ops

    fx = _fixture(name)
    p = fx["params"]
    mtp = p["mtp"]
    print(f"GOLDEN {name} params={p}", flush=True)
    d = make_golden.build_case(p).to_device("cuda")
    t = d.tensors
    lim_args = (t["query_index"], t["index_weights"], t["index_key_cache"], t["index_block_table"],
                t["num_candidate_tokens"], t["num_cache_tokens"], t["req_pool_entries"], t["cache_slots_pool"],
                t["topk_src_ids"], t["topk_dst_slots"])
    if mtp:
        ops.fused_li_manage_mtp(*lim_args, t["miss_src_ids"], t["miss_dst_slots"], t["miss_counts"])
    else:
        ops.fused_li_manage(*lim_args, t["miss_counts"])
    torch.cuda.synchronize()
    got = dict(src=ints(t["topk_src_ids"]), dst=ints(t["topk_dst_slots"]), miss_counts=ints(t["miss_counts"]),
               pool=ints(t["cache_slots_pool"]))
    if mtp:
        got["miss_src"] = ints(t["miss_src_ids"])
        got["miss_dst"] = ints(t["miss_dst_slots"])
    for key, val in got.items():
        assert np.array_equal(val, fx[key]), (name, key)

    out = t["attention_out"]
    out.fill_(7.0)
    common = (t["query_rope"], t["query"], t["actual_seq_lengths_query"], t["actual_seq_lengths_kv"],
              t["num_cache_tokens"], t["topk_dst_slots"])
    caches = (t["hbm_block_table"], t["dram_block_table"], t["hbm_k_rope"], t["hbm_kv_cache"], t["dram_k_rope"],
              t["dram_kv_cache"], d.meta["scale"], out)
    if mtp:
        ops.fused_copy_sfa_mtp(*common, t["topk_src_ids"], t["miss_src_ids"], t["miss_dst_slots"], t["miss_counts"],
                               *caches)
    else:
        B = t["query"].shape[0]
        ops.fused_copy_sfa(*common, t["topk_src_ids"].view(B, -1), t["miss_counts"], *caches)
    torch.cuda.synchronize()
    assert make_golden.digest(bits(t["hbm_kv_cache"])) == fx["hbm_kv_digest"], name
    assert make_golden.digest(bits(t["hbm_k_rope"])) == fx["hbm_kpe_digest"], name
    assert_attention_close(out, fx["attention"].astype(np.float64), t["query"].dtype, label=f"golden {name}")
