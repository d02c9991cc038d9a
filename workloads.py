"""Synthetic LLaMA-7B / PointLLM-7B inputs for the W8A8 projections.

Shapes come from the reference's PointLLM workload description
(architecture_simulator/pointllm_archsim/workload.py:31-35: hidden 4096,
intermediate 11008, vocab 32003, 513 point tokens) and the packed QKV /
gate-up layouts (llama/paged_attention.py:1242-1245,
llama/lightweight_runner.py:57-93).  There is no network, so weights are
random-initialised ~N(0, 0.02) and activations are seeded normals with
outlier channels, generated on the CPU with ``torch.Generator`` (the same
values on every machine) unless a device generator is requested.

Bench and test support (bench.py, __graft_entry__.smoke and tests/), kept
outside the nanopointllm_amd package: nothing in the package imports it.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

HIDDEN = 4096
INTERMEDIATE = 11008
HEADS = 32
KV_HEADS = 32
HEAD_DIM = 128
VOCAB = 32003
LAYERS = 32
POINT_TOKENS = 513


@dataclass(frozen=True)
class Projection:
    name: str
    n: int          # packed output rows
    k: int          # input features
    silu: bool      # packed interleaved gate/up with fused SiLU*mul (outputs n/2)


PROJECTIONS = (
    Projection("qkv", 3 * HIDDEN, HIDDEN, False),
    Projection("o", HIDDEN, HIDDEN, False),
    Projection("gateup", 2 * INTERMEDIATE, HIDDEN, True),
    Projection("down", HIDDEN, INTERMEDIATE, False),
)


def algorithmic_bytes(m: int, n: int, k: int, *, silu: bool = False, int8_in: bool = False,
                      int8_out: bool = False) -> int:
    """Bytes a W8A8 linear must move: int8 W + fp16 s_w + activations in/out.

    ``N*K + 2N + 2MK + 2M*N_out`` (N_out = N/2 with SiLU*mul); an int8 input
    counts ``M*K + 4M`` and an int8 output ``M*N_out + 4M``.
    """
    n_out = n // 2 if silu else n
    b = n * k + 2 * n
    b += (m * k + 4 * m) if int8_in else 2 * m * k
    b += (m * n_out + 4 * m) if int8_out else 2 * m * n_out
    return b


def algorithmic_ops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def _gen(seed: int, device: str | torch.device = "cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def decode_activations(m: int, k: int, *, seed: int = 0, outliers: int = 8,
                       dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """~N(0, 1) rows with `outliers` channels scaled x20 (CPU, seeded).

    Draw order: ``randn(m, k)``, then ``randperm(k)[:outliers]`` from the same
    generator.
    """
    g = _gen(seed)
    x = torch.randn(m, k, generator=g)
    idx = torch.randperm(k, generator=g)[:outliers]
    x[:, idx] *= 20.0
    return x.to(dtype)


def prefill_activations(m: int, k: int, *, seed: int = 0, point_tokens: int = POINT_TOKENS,
                        dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Point-token rows ~N(0, 0.5), text rows ~N(0, 1), 0.1% of channels x20."""
    g = _gen(seed)
    x = torch.randn(m, k, generator=g)
    x[:point_tokens] *= 0.5
    n_out = max(1, round(k * 0.001))
    idx = torch.randperm(k, generator=g)[:n_out]
    x[:, idx] *= 20.0
    return x.to(dtype)


def linear_weight(n: int, k: int, *, seed: int = 1, dtype: torch.dtype = torch.float16,
                  device: str | torch.device = "cpu") -> torch.Tensor:
    """~N(0, 0.02) weight, drawn in f32 and stored as `dtype`."""
    g = _gen(seed, device)
    return (torch.randn(n, k, generator=g, device=device) * 0.02).to(dtype)


def config1(seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Single W8A8 linear: X fp16 [16, 4096] (8 outlier channels), W [4096, 4096]."""
    g = _gen(seed)
    x = torch.randn(16, HIDDEN, generator=g)
    idx = torch.randperm(HIDDEN, generator=g)[:8]
    x[:, idx] *= 20.0
    w = torch.randn(HIDDEN, HIDDEN, generator=g) * 0.02
    return x.to(torch.float16), w.to(torch.float16)


class RMSNorm(nn.Module):
    """``LightweightRMSNorm`` (lightweight_runner.py:239-245): binary32 mean of
    squares, ``rsqrt(var + eps)``, cast back, times the weight."""

    def __init__(self, hidden: int, eps: float = 1e-6, *, device=None, dtype=None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden, device=device, dtype=dtype))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        h = x.float()
        var = h.pow(2).mean(-1, keepdim=True)
        h = h * torch.rsqrt(var + self.variance_epsilon)
        return self.weight * h.to(dtype)


class _Attention(nn.Module):
    def __init__(self, hidden: int, heads: int, kv_heads: int, **kw) -> None:
        super().__init__()
        self.num_heads, self.num_key_value_heads = heads, kv_heads
        self.head_dim = hidden // heads
        kv = kv_heads * self.head_dim
        self.q_proj = nn.Linear(hidden, hidden, bias=False, **kw)
        self.k_proj = nn.Linear(hidden, kv, bias=False, **kw)
        self.v_proj = nn.Linear(hidden, kv, bias=False, **kw)
        self.o_proj = nn.Linear(hidden, hidden, bias=False, **kw)


class _MLP(nn.Module):
    def __init__(self, hidden: int, intermediate: int, **kw) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(hidden, intermediate, bias=False, **kw)
        self.up_proj = nn.Linear(hidden, intermediate, bias=False, **kw)
        self.down_proj = nn.Linear(intermediate, hidden, bias=False, **kw)


class _DecoderLayer(nn.Module):
    def __init__(self, hidden: int, heads: int, kv_heads: int, intermediate: int, **kw) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(hidden, **kw)
        self.self_attn = _Attention(hidden, heads, kv_heads, **kw)
        self.post_attention_layernorm = RMSNorm(hidden, **kw)
        self.mlp = _MLP(hidden, intermediate, **kw)


class LlamaShaped(nn.Module):
    """The module tree of a Hugging Face ``LlamaForCausalLM`` that the
    reference's runners read (``model.embed_tokens``, ``model.layers[i]``
    with ``input_layernorm`` / ``self_attn.{q,k,v,o}_proj`` /
    ``post_attention_layernorm`` / ``mlp.{gate,up,down}_proj``,
    ``model.norm``, ``lm_head``; lightweight_runner.py:421-737), with no
    forward of its own: the W8A8 runner supplies it."""

    def __init__(self, *, hidden: int = HIDDEN, heads: int = HEADS, kv_heads: int = KV_HEADS,
                 intermediate: int = INTERMEDIATE, vocab: int = VOCAB, layers: int = LAYERS,
                 device=None, dtype=None) -> None:
        super().__init__()
        kw = {"device": device, "dtype": dtype}
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(vocab, hidden, **kw)
        self.model.layers = nn.ModuleList([_DecoderLayer(hidden, heads, kv_heads, intermediate,
                                                         **kw) for _ in range(layers)])
        self.model.norm = RMSNorm(hidden, **kw)
        self.lm_head = nn.Linear(hidden, vocab, bias=False, **kw)


def llama_model(device: str | torch.device, *, layers: int = LAYERS, seed: int = 0,
                dtype: torch.dtype = torch.float16, **shape) -> LlamaShaped:
    """A LLaMA-7B-shaped model (``shape`` overrides hidden / heads / kv_heads /
    intermediate / vocab) with random weights drawn on ``device``: linear
    weights ~N(0, 0.02), norm weights 1 + N(0, 0.1), embeddings ~N(0, 1).
    The parameters are created without initialisation and filled once."""
    with torch.device("meta"):
        model = LlamaShaped(layers=layers, dtype=dtype, **shape)
    model = model.to_empty(device=device)
    g = _gen(seed, device)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.normal_(1.0, 0.1, generator=g)
            elif "embed" in name:
                p.normal_(0.0, 1.0, generator=g)
            else:
                p.normal_(0.0, 0.02, generator=g)
    return model


def query_passthrough_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_index: int,
                           state) -> torch.Tensor:
    """A stand-in for the attention core that returns the query rows as the
    context ``[T, H * D]`` (a view, no kernel): the step around it is the
    W8A8 path alone.  Rotary, the KV cache and the attention kernel are not
    part of that path."""
    return q.reshape(q.shape[0], -1)
