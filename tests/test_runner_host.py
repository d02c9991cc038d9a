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


def _bare_runner(norm):
    from nanopointllm_amd.runner import W8A8LlamaRunner

    runner = W8A8LlamaRunner.__new__(W8A8LlamaRunner)
    nn.Module.__init__(runner)
    runner.norm = norm
    return runner


def test_final_norm_routing():
    """Binary32 rows (or a norm weight of another dtype) run the model's own
    norm module on dtype(hidden + residual); 16-bit rows with a matching
    weight go to the activation prologue kernel, which has no host path."""
    from nanopointllm_amd.workloads import RMSNorm

    norm = RMSNorm(8)
    with torch.no_grad():
        norm.weight.copy_(torch.linspace(0.5, 1.5, 8))
    runner = _bare_runner(norm)
    h, r = torch.randn(3, 8), torch.randn(3, 8)
    with torch.no_grad():
        assert torch.equal(runner.final_norm(h, r), norm(r + h))
        assert torch.equal(runner.final_norm(h, None), norm(h))
    half = _bare_runner(RMSNorm(8, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="only on the GPU"):
        half.final_norm(h.half(), r.half())
