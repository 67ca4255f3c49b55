"""Capture-size rules of nanovllm_amd.decode_graph (CPU): the reference's
normalize_capture_sizes / select_capture_size
(nanovllm/engine/full_decode_graph.py:33-57) and the runtime-input checks of
DsaLayerGraph (shape errors are raised before any GPU work)."""

from __future__ import annotations

import pytest


def test_normalize_capture_sizes():
    from nanovllm_amd.decode_graph import normalize_capture_sizes

    assert normalize_capture_sizes([16, 4, 8, 4]) == (4, 8, 16)
    with pytest.raises(ValueError, match="at least one"):
        normalize_capture_sizes([])
    with pytest.raises(ValueError, match="must be positive"):
        normalize_capture_sizes([0, 8])


def test_select_capture_size():
    from nanovllm_amd.decode_graph import select_capture_size

    sizes = (4, 8, 16)
    assert select_capture_size(1, sizes) == 4
    assert select_capture_size(4, sizes) == 4
    assert select_capture_size(5, sizes) == 8
    assert select_capture_size(16, sizes) == 16
    assert select_capture_size(17, sizes) is None
