"""W8A8 injection into a small LLaMA-shaped model (the structure of the
reference's fake HF model, tests/test_lightweight_runner.py:8-75, at sizes
that exercise the packed layouts)."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, INTER = 256, 4, 384


def note(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.num_heads = HEADS
        self.num_key_value_heads = HEADS
        self.head_dim = HIDDEN // HEADS
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self, name, nn.Linear(HIDDEN, HIDDEN, bias=False))


class _MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(HIDDEN, INTER, bias=False)
        self.up_proj = nn.Linear(HIDDEN, INTER, bias=False)
        self.down_proj = nn.Linear(INTER, HIDDEN, bias=False)
        self.act_fn = F.silu

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Attn()
        self.mlp = _MLP()


class _FakeLlama(nn.Module):
    def __init__(self, layers=2):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([_Layer() for _ in range(layers)])


def _model(device):
    torch.manual_seed(0)
    m = _FakeLlama()
    with torch.no_grad():
        for p in m.parameters():
            p.mul_(0.5)
    return m.to(device=device, dtype=torch.float16)


def _oracle_linear(x16, w16):
    _, q, s = O.per_output_weight_qdq(w16.float().cpu().numpy())
    out, _, _, _ = O.w8a8_linear_dynamic(x16.float().cpu().numpy().reshape(-1, w16.shape[1]), q, s)
    return out.astype(np.float16)


def test_inject_replaces_all_projections(cuda):
    from nanopointllm_amd.inject import inject_w8a8
    from nanopointllm_amd.linear import W8A8Linear

    model = _model(cuda)
    dense = {n: p.detach().clone() for n, p in model.named_parameters()}
    note("inject fake llama")
    counts = inject_w8a8(model)
    assert counts == {"linear": 14, "packed_qkv": 2, "packed_mlp": 2}
    layer = model.model.layers[1]
    assert isinstance(layer.self_attn.o_proj, W8A8Linear)
    assert isinstance(layer.mlp.down_proj, W8A8Linear)
    x = (torch.randn(3, HIDDEN, generator=torch.Generator().manual_seed(1)) * 2).to(torch.float16)
    for name in ("q_proj", "o_proj"):
        got = getattr(layer.self_attn, name)(x.to(cuda)).cpu().numpy()
        exp = _oracle_linear(x, dense[f"model.layers.1.self_attn.{name}.weight"])
        np.testing.assert_array_equal(got, exp)
    # second injection is a no-op
    assert inject_w8a8(model) == {"linear": 0, "packed_qkv": 0, "packed_mlp": 0}


def test_packed_call_site_helpers(cuda):
    from nanopointllm_amd.inject import (inject_w8a8, packed_mlp_decode,
                                         project_output_decode_staged,
                                         project_qkv_decode_packed)

    model = _model(cuda)
    inject_w8a8(model)
    layer = model.model.layers[0]
    hs = (torch.randn(1, 5, HIDDEN, generator=torch.Generator().manual_seed(2))).to(torch.float16).to(cuda)
    note("packed qkv helper")
    q, k, v = project_qkv_decode_packed(hs, layer.self_attn.w8a8_qkv)
    assert q.shape == (5, HEADS, HIDDEN // HEADS) and k.shape == v.shape == q.shape
    torch.testing.assert_close(q.reshape(5, -1), layer.self_attn.q_proj(hs[0]), rtol=0, atol=0)
    torch.testing.assert_close(v.reshape(5, -1), layer.self_attn.v_proj(hs[0]), rtol=0, atol=0)
    note("o proj helper")
    o = project_output_decode_staged(hs, layer.self_attn.o_proj)
    assert o.shape == (1, 5, HIDDEN)
    note("packed mlp helper")
    y = packed_mlp_decode(hs, layer.mlp.w8a8_mlp)
    assert y.shape == (1, 5, HIDDEN)
    h = layer.mlp.w8a8_mlp.gate_up(hs[0])
    torch.testing.assert_close(y[0], layer.mlp.w8a8_mlp.down(h), rtol=0, atol=0)
    assert torch.isfinite(y).all()
