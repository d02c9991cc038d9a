"""Host-side behaviour of the W8A8 decoder stack (runner.py) that needs no GPU:
argument validation, the injection requirement and the graph bucket's state
checks (the reference's strict wrapper raises the same way,
nanopointllm/engine/cuda_graph.py:30-52)."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn


def test_rows_layout_validation():
    from nanopointllm_amd.runner import _rows

    x = torch.randn(1, 5, 8)
    assert _rows(x).shape == (5, 8)
    assert _rows(torch.randn(5, 8)).shape == (5, 8)
    assert _rows(x.transpose(1, 2).transpose(1, 2)).is_contiguous()
    with pytest.raises(ValueError):
        _rows(torch.randn(2, 5, 8))
    with pytest.raises(ValueError):
        _rows(torch.randn(8))


def test_layer_without_w8a8_modules_is_rejected():
    from nanopointllm_amd.runner import W8A8LlamaLayer

    layer = nn.Module()
    layer.self_attn = nn.Module()
    layer.self_attn.o_proj = nn.Linear(4, 4)
    layer.mlp = nn.Module()
    with pytest.raises(ValueError, match="inject_w8a8"):
        W8A8LlamaLayer(layer, 0, lambda q, k, v, i, s: q)


def test_graph_bucket_state_checks():
    from nanopointllm_amd.runner import DecodeGraphBucket

    bucket = DecodeGraphBucket("cpu")
    assert not bucket.captured
    with pytest.raises(RuntimeError, match="not been captured"):
        bucket.replay()
    with pytest.raises(RuntimeError, match="needs a GPU"):
        bucket.capture(lambda: torch.zeros(1))
