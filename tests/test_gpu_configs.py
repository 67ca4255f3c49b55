"""Every BASELINE.json configuration at its full size on the GPU vs the oracle.

Each test builds the configuration's whole workload with the no-near-tie
guard (nanovllm_amd.workloads.baseline_config), runs the oracle once, and then
runs the HIP chain through the reference-signature wrappers:

* ``fused_li_manage(_mtp)``: top-k ids, slots, miss lists and counts, and the
  updated slot pool bit-exact;
* then offload_fuse (``fused_copy_sfa(_mtp)``) and offload_split
  (``scatter_copy`` -> ``sparse_tail_attention(_mtp)``, glm_mla.py:1298,
  :1317, :1847): both HBM caches after the copy bit-exact and the attention
  within the north-star tolerance (max-abs 2e-2, mean-rel 1e-3 vs the golden
  rounded to bf16);
* at the tables' natural width and at the model runner's layout: every
  block table padded with 0 to 512 columns and a 65536-wide pool
  (max_model_len 65536; nanovllm/engine/model_runner.py:587-598, :747-752),
  which the LIM sees as S_cap = 65536.

cfg0: bs=1, 20480 tokens, tail 37.  cfg1: bs=24, 32768, tails U[1,127].
cfg2: bs=64, U[20K,64K].  cfg3: MTP3 bs=16 x 4, 49152, C=8192.
cfg4 (the 78-layer IndexShare step) is in test_gpu_index_share_full.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _chain import (check_copy_attend, check_lim, oracle_chain, poison_outputs, run_copy_attend, run_lim,
                    widen_layout)
from _helpers import ints, oracle_lim

pytestmark = pytest.mark.gpu

CALLER_CAPACITY = 65536
MUTABLE = ("cache_slots_pool", "hbm_kv_cache", "hbm_k_rope")


def _run_config(index: int, layouts, paths) -> None:
    from nanovllm_amd.workloads import baseline_config

    case = baseline_config(index, seed=index, guard=True)
    mtp = case.meta["mtp"]
    print(f"CFG{index} built: B={case.meta['batch']} halvings={case.meta['halvings']} "
          f"miss_target={sum(case.meta['miss_target'])}", flush=True)
    lim = oracle_lim(case, mtp=mtp)
    gold, hkpe, hckv = oracle_chain(case, lim, mtp)
    print(f"CFG{index} oracle: misses={int(lim['miss_counts'].sum())}", flush=True)
    assert int(lim["miss_counts"].sum()) > 0
    d = case.to_device("cuda")
    base = d.tensors
    init = {k: base[k].clone() for k in MUTABLE}
    cap0 = base["cache_slots_pool"].shape[1]
    for layout in layouts:
        t = dict(base)
        for k in MUTABLE:
            t[k] = init[k].clone()
        if layout is not None:
            t = widen_layout(t, layout, pad=0)
        wide_init = ints(t["cache_slots_pool"])
        for path in paths:
            label = f"cfg{index} S_cap={t['cache_slots_pool'].shape[1]} {path}"
            t["cache_slots_pool"].copy_(torch.from_numpy(wide_init))
            t["hbm_kv_cache"].copy_(init["hbm_kv_cache"])
            t["hbm_k_rope"].copy_(init["hbm_k_rope"])
            poison_outputs(t, mtp)
            torch.cuda.synchronize()
            print(f"RUN {label}: LIM", flush=True)
            run_lim(t, mtp)
            torch.cuda.synchronize()
            check_lim(t, lim, mtp, label, pool_cols=cap0)
            assert np.array_equal(ints(t["cache_slots_pool"])[:, cap0:], wide_init[:, cap0:]), label
            print(f"RUN {label}: copy + attention", flush=True)
            run_copy_attend(t, case.meta["scale"], mtp, fused=path == "fused")
            torch.cuda.synchronize()
            check_copy_attend(t, gold, hkpe, hckv, label)
    del d, base, init
    torch.cuda.empty_cache()


def test_cfg0_bs1_20480_tail37():
    _run_config(0, (None, CALLER_CAPACITY), ("split", "fused"))


def test_cfg1_bs24_32k():
    _run_config(1, (None, CALLER_CAPACITY), ("fused", "split"))


def test_cfg2_bs64_mixed_20k_64k():
    _run_config(2, (None, CALLER_CAPACITY), ("fused", "split"))


def test_cfg3_mtp3_bs16x4_48k():
    _run_config(3, (None, CALLER_CAPACITY), ("fused", "split"))
