"""Write tests/golden/chain_golden.npz: expected outputs of the oracle chain
(LIM -> copy -> attention) on small seeded workloads.

The inputs are not stored: ``nanovllm_amd.workloads.make_chain_case`` rebuilds
them bit for bit from the parameters kept beside the outputs (seeded CPU torch
generators).  The reference holds no fixture files for this path (its op tests
generate their goldens from seeds too), so these vectors are this build's own:
they freeze the oracle's canonical results so that a later change of the
oracle or of the generator shows up as a test failure, and they give the GPU
tests expected outputs that do not depend on running the oracle.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
for p in (REPO / "nanovllm-dsa-offload_amd", REPO, HERE.parent):
    sys.path.insert(0, str(p))

import torch  # noqa: E402

from oracle import dsa_oracle as O  # noqa: E402

CASES = {
    "mtp0_bf16": dict(batch=2, source_lens=[2560, 4096], cache_tokens=[2048, 2560], tails=[37, 90], seed=101,
                      index_heads=32, attn_heads=16, dtype="bf16", mtp=False),
    "mtp0_f16_h64": dict(batch=1, source_lens=[3072], cache_tokens=[2048], tails=[5], seed=102, index_heads=64,
                         attn_heads=16, dtype="f16", mtp=False),
    "mtp3_bf16": dict(batch=1, source_lens=[9216], cache_tokens=[8192], tails=[6], seed=103, index_heads=32,
                      attn_heads=16, dtype="bf16", mtp=True),
}


def build_case(params: dict):
    from nanovllm_amd.workloads import make_chain_case

    dtype = torch.bfloat16 if params["dtype"] == "bf16" else torch.float16
    return make_chain_case(params["batch"], params["source_lens"], params["cache_tokens"], params["tails"],
                           index_heads=params["index_heads"], attn_heads=params["attn_heads"], seed=params["seed"],
                           dtype=dtype, mtp=params["mtp"])


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_oracle(case, mtp: bool) -> dict:
    """Oracle LIM, then the fused copy + attention on its outputs."""
    from _helpers import bits, dname, ints, oracle_lim

    lim = oracle_lim(case, mtp=mtp)
    t = case.tensors
    dt = dname(t["query"].dtype)
    hkpe, hckv = bits(t["hbm_k_rope"]), bits(t["hbm_kv_cache"])
    common = (bits(t["query_rope"]), bits(t["query"]), ints(t["actual_seq_lengths_kv"]), ints(t["num_cache_tokens"]),
              lim["dst"])
    tail = (ints(t["hbm_block_table"]), ints(t["dram_block_table"]), hkpe, hckv, bits(t["dram_k_rope"]),
            bits(t["dram_kv_cache"]), case.meta["scale"])
    if mtp:
        out = O.fused_copy_sfa_mtp(*common, lim["miss_src"], lim["miss_dst"], lim["miss_counts"], *tail, dtype=dt)
    else:
        B = t["query"].shape[0]
        out = O.fused_copy_sfa(*common, lim["src"].reshape(B, O.TOPK), lim["miss_counts"], *tail, dtype=dt)
    res = dict(lim)
    res["attention"] = np.asarray(out, np.float32)
    res["hbm_kv_digest"] = digest(hckv)
    res["hbm_kpe_digest"] = digest(hkpe)
    return res


def main() -> None:
    arrays = {}
    for name, params in CASES.items():
        res = run_oracle(build_case(params), params["mtp"])
        arrays[f"{name}/params"] = np.frombuffer(json.dumps(params, sort_keys=True).encode(), dtype=np.uint8)
        for key, val in res.items():
            if isinstance(val, str):
                arrays[f"{name}/{key}"] = np.frombuffer(val.encode(), dtype=np.uint8)
            else:
                arrays[f"{name}/{key}"] = val
        print(name, "misses", res["miss_counts"].tolist(), flush=True)
    np.savez_compressed(HERE / "chain_golden.npz", **arrays)
    print("wrote", HERE / "chain_golden.npz")


if __name__ == "__main__":
    main()
