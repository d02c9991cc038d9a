"""Synthetic LLaMA-7B / PointLLM-7B inputs for the W8A8 projections.

Shapes come from the reference's PointLLM workload description
(architecture_simulator/pointllm_archsim/workload.py:31-35: hidden 4096,
intermediate 11008, vocab 32003, 513 point tokens) and the packed QKV /
gate-up layouts (llama/paged_attention.py:1242-1245,
llama/lightweight_runner.py:57-93).  There is no network, so weights are
random-initialised ~N(0, 0.02) and activations are seeded normals with
outlier channels, generated on the CPU with ``torch.Generator`` (the same
values on every machine) unless a device generator is requested.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

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
