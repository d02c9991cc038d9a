"""Torch-CPU restatement of the reference's integer linear path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module: it is the CPU path that the benchmark
times next to the GPU (the reference's own golden runs these torch calls on
the CPU), and a second oracle to compare results with.  The product path
under ``nano-pointllm_amd/`` never imports it.

It follows the reference's torch code step by step, on CPU tensors:

* ``scale_from_absmax``   - nanopointllm/compression/w8a8.py:46-50
* ``quantize_symmetric``  - w8a8.py:33-43 (``torch.round`` ties to even,
  clamp to [-127, 127])
* ``per_token_linear``    - dynamic per-token activation scale (w8a8.py:
  106-115) feeding ``integer_linear_per_output_reference`` (w8a8.py:118-139):
  int32 ``flat @ qweight.T`` on the CPU, then ``out *= s_x; out *= s_w;
  out += bias`` in binary32
* ``silu_mul``            - ``act_fn(gate) * up`` of the packed MLP on binary16
  tensors (llama/lightweight_runner.py:344-358), gate/up split from the
  interleaved packed output

Pinned in tests/test_oracle.py against the numpy oracle (itself pinned by the
reference's KATs): scales, int8 values, int32 accumulators and binary32
outputs bit-equal on random inputs with outlier channels, and the reference's
tiny int32 linear KAT (tests/test_w8a8_contract.py:55-76).
"""
from __future__ import annotations

import torch

SYMMETRIC_MIN, SYMMETRIC_MAX = -127, 127


def scale_from_absmax(absmax: torch.Tensor) -> torch.Tensor:
    """w8a8.py:46-50: binary16-stored scale, returned in binary32."""
    tiny = torch.finfo(torch.float16).tiny
    raw = absmax.float().clamp_min(tiny) / SYMMETRIC_MAX
    return raw.to(torch.float16).float().clamp_min(tiny)


def quantize_symmetric(values: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """w8a8.py:33-43 (the positivity check is the caller's)."""
    q = torch.round(values.float() / scale.float()).clamp(SYMMETRIC_MIN, SYMMETRIC_MAX)
    return q.to(torch.int8)


def per_token_linear(values: torch.Tensor, qweight: torch.Tensor, weight_scales: torch.Tensor,
                     bias: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token A8 x per-output W8 linear of the reference's CPU golden.

    ``values`` [M, K] (any float dtype), ``qweight`` int8 [N, K],
    ``weight_scales`` binary32 [N].  Returns ``(out f32 [M, N], acc int32)``.
    """
    scales = scale_from_absmax(values.detach().float().abs().amax(dim=-1, keepdim=True))
    qactivation = quantize_symmetric(values, scales)
    accumulator = qactivation.to(torch.int32) @ qweight.to(torch.int32).transpose(0, 1)
    output = accumulator.float()
    output *= scales
    output *= weight_scales.float().unsqueeze(0)
    if bias is not None:
        output += bias.float().unsqueeze(0)
    return output, accumulator


def silu_mul(gate_up16: torch.Tensor) -> torch.Tensor:
    """``act_fn(gate) * up`` on the binary16 packed gate/up output in the
    interleaved row order (lightweight_runner.py:344-358)."""
    pairs = gate_up16.view(*gate_up16.shape[:-1], gate_up16.shape[-1] // 2, 2)
    return torch.nn.functional.silu(pairs[..., 0]) * pairs[..., 1]
