"""IndexShare topology and step ordering, CPU only.

The GLM-5.2 schedule and group manager against the reference's expectations
(tests/test_glm_index_share.py:112-260 of the reference: 21 groups over 78
layers, owners 0, 1, 2, 6, 10, ..., 74, the last group 74-77, GLM-5.1
degrading to one group per layer, and the error cases), with the expected
owner list derived here by walking the schedule rule rather than from the
code under test; and the driver's refusal to run a shared layer before its
owner in a step.
"""

from __future__ import annotations

import pytest
import torch

from nanovllm_amd.index_share import (DsaLayerCaches, IndexShareDecodeStep, IndexShareGroup, IndexShareGroupManager,
                                      glm52_indexer_types)


def test_glm52_schedule_21_owners_57_shared():
    types = glm52_indexer_types(78)
    mgr = IndexShareGroupManager(78, types)
    owners = (0, 1, 2) + tuple(range(6, 78, 4))
    assert mgr.num_groups == 21 and mgr.owner_layer_idxs == owners
    assert len(mgr.shared_layer_idxs) == 57
    assert mgr.shared_layer_idxs == tuple(i for i in range(78) if i not in owners)
    assert mgr.group(0) == IndexShareGroup(0, 0, (0,))
    assert mgr.group(1) == IndexShareGroup(1, 1, (1,))
    assert mgr.group(2) == IndexShareGroup(2, 2, (2, 3, 4, 5))
    assert mgr.group(20) == IndexShareGroup(20, 74, (74, 75, 76, 77))
    members = [m for g in mgr.groups() for m in g.member_layer_idxs]
    assert sorted(members) == list(range(78)) and len(members) == 78


def test_glm52_owner_and_group_mapping():
    mgr = IndexShareGroupManager(78, glm52_indexer_types(78))
    for layer, owner in ((3, 2), (4, 2), (5, 2), (7, 6), (9, 6), (75, 74), (77, 74)):
        assert mgr.owner_of(layer) == owner and mgr.is_shared(layer) and not mgr.is_owner(layer)
    for owner in mgr.owner_layer_idxs:
        assert mgr.owner_of(owner) == owner and mgr.is_owner(owner) and not mgr.is_shared(owner)
    for g in mgr.groups():
        for layer in g.member_layer_idxs:
            assert mgr.group_of(layer) == g.group_id
    assert [g.group_id for g in mgr.groups()] == list(range(21))


def test_glm51_degrades_to_single_layer_groups():
    mgr = IndexShareGroupManager(78)
    assert mgr.num_groups == 78 and mgr.shared_layer_idxs == ()
    assert all(mgr.owner_of(i) == i and mgr.group(i).member_layer_idxs == (i,) for i in range(78))


@pytest.mark.parametrize("types,match", [
    (("full", "shared"), "length must match"),
    (("shared", "full", "full"), "no preceding full layer"),
    (("full", "dense", "full"), "Unknown indexer_type"),
])
def test_group_manager_errors(types, match):
    with pytest.raises(ValueError, match=match):
        IndexShareGroupManager(3, types)


def test_group_manager_validate_layer():
    mgr = IndexShareGroupManager(4, ("full", "shared", "full", "shared"))
    mgr.validate_layer(3)
    with pytest.raises(IndexError):
        mgr.validate_layer(4)


def _caches(owner: bool) -> DsaLayerCaches:
    z = torch.zeros(1, 128, 1, 8)
    extra = dict(index_key_cache=torch.zeros(1), cache_slots_pool=torch.zeros(1, 128, dtype=torch.int32)) if owner else {}
    return DsaLayerCaches(z, z, z, z, **extra)


def test_step_refuses_shared_layer_before_owner_and_missing_owner_state():
    mgr = IndexShareGroupManager(2, ("full", "shared"))
    with pytest.raises(ValueError, match="owner layer 0"):
        IndexShareDecodeStep(mgr, [_caches(False), _caches(False)])
    with pytest.raises(ValueError, match="expected 2 layers"):
        IndexShareDecodeStep(mgr, [_caches(True)])
    runner = IndexShareDecodeStep(mgr, [_caches(True), _caches(False)])
    ctx = {"num_candidate_tokens": torch.zeros(3, dtype=torch.int32)}
    with pytest.raises(RuntimeError, match="before its owner"):
        runner.run_layer(1, ctx, query_rope=None, query=None, scale=1.0, attention_out=None)
    with pytest.raises(RuntimeError, match="requires indexer outputs"):
        runner.run_layer(0, ctx, query_rope=None, query=None, scale=1.0, attention_out=None)
    out = runner.owner_outputs(0, 3)
    assert out["topk_src_ids"].shape == (3, 1, 2048) and out["miss_counts"].shape == (3,)
    assert runner.owner_outputs(0, 3)["topk_dst_slots"] is out["topk_dst_slots"]  # fixed addresses
    with pytest.raises(ValueError, match="missing"):
        runner.step({}, lambda i: {})
