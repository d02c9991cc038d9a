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
    from workloads import RMSNorm

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


def test_rows2_and_norm_eps_refuse_what_they_cannot_serve():
    """The staged-decode helpers take ``[1, T, H]`` or ``[T, H]`` only (a
    batch other than 1 would silently drop rows), and a norm without an
    epsilon attribute is refused rather than given a default."""
    from types import SimpleNamespace

    from nanopointllm_amd.linear import _norm_eps, _rows2

    assert _rows2(torch.zeros(1, 5, 8)).shape == (5, 8)
    assert _rows2(torch.zeros(5, 8)).shape == (5, 8)
    with pytest.raises(ValueError, match="tokens, hidden"):
        _rows2(torch.zeros(2, 5, 8))
    with pytest.raises(ValueError, match="tokens, hidden"):
        _rows2(torch.zeros(8))
    assert _norm_eps(SimpleNamespace(variance_epsilon=1e-5)) == 1e-5
    assert _norm_eps(SimpleNamespace(eps=3e-6)) == 3e-6
    with pytest.raises(ValueError, match="no epsilon"):
        _norm_eps(SimpleNamespace(weight=None))


def test_fused_norm_mlp_keeps_the_plain_chain_with_two_phase(monkeypatch):
    """``W8A8MLP.forward_residual_rmsnorm`` hands the fused norm + gate/up
    launch's 16-bit h to down's own per-token quantization whether or not
    ``two_phase`` is set (same bits either way); the two-phase gate/up is
    not called."""
    from types import SimpleNamespace

    from nanopointllm_amd import _lib, linear

    calls = []

    def fake_rmsnorm_linear(x, w, eps, packed, scale, bias, n, **kw):
        calls.append(("rmsnorm_linear", kw.get("epilogue"), kw.get("residual") is not None))
        return SimpleNamespace(y="h", residual="summed")

    monkeypatch.setattr(linear._w, "rmsnorm_linear", fake_rmsnorm_linear)
    for two_phase in (False, True):
        calls.clear()
        mlp = linear.W8A8MLP.__new__(linear.W8A8MLP)
        nn.Module.__init__(mlp)
        mlp.gate_up = SimpleNamespace(
            weight_q=SimpleNamespace(packed=None, scale=None, bias=None, out_features=16,
                                     in_features=8),
            forward_two_phase=lambda *a, **k: calls.append("two_phase"))
        mlp.down = lambda h: calls.append(("down", h)) or "y"
        mlp.h_scale = None
        mlp.two_phase = two_phase
        norm = SimpleNamespace(weight=None, variance_epsilon=1e-6)
        out = mlp.forward_residual_rmsnorm("x", "r", norm)
        assert out == ("summed", "y")
        assert calls == [("rmsnorm_linear", _lib.EPI_SILU_MUL, True), ("down", "h")]
