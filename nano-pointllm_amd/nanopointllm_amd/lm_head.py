"""The LM head at decode batches (``w8a8_dense_gemv`` of libw8a8_gfx950.so).

The reference's LM head is a plain 16-bit ``nn.Linear``; at decode it runs as
``F.linear`` of the final-norm rows (``_decode_linear_rows`` /
``_decode_staged_linear``, nanopointllm/llama/lightweight_runner.py:38-43,
96-99, 676-681).  ``dense_gemv`` computes the same product for up to 16 rows
with a hand-written gfx950 kernel that streams the module's own row-major
weight once (binary32 accumulation, one rounding to the output type, a fixed
summation order, so a row's logits do not depend on the other rows of the
batch).  ``DecodeLMHead`` wraps the module: decode batches take the kernel,
larger batches keep the module's own GEMM (``F.linear``), as the reference
does for prefill.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib

MAX_ROWS = 16
MAX_K = 8192


def dense_gemv_supported(x: torch.Tensor, weight: torch.Tensor,
                         bias: torch.Tensor | None = None) -> bool:
    """Whether ``dense_gemv`` takes these operands (else it raises)."""
    if not (x.is_cuda and weight.is_cuda) or x.dtype not in (torch.float16, torch.bfloat16):
        return False
    if weight.dtype != x.dtype or weight.dim() != 2 or weight.stride(-1) != 1:
        return False
    if bias is not None and (bias.dtype != x.dtype or bias.dim() != 1 or not bias.is_contiguous()):
        return False
    k = x.shape[-1]
    rows = x.numel() // k if k else 0
    return (weight.shape[1] == k and 1 <= rows <= MAX_ROWS and 0 < k <= MAX_K and k % 8 == 0
            and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0)


def dense_gemv(x: torch.Tensor, weight: torch.Tensor,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` for at most 16 rows of 16-bit x on the GPU.

    x [..., K] and weight [N, K] (row-major, unit column stride) share a
    16-bit dtype; the result [..., N] has it too.
    """
    device = _lib.require_cuda(x, weight, bias)
    if x.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != x.dtype:
        raise ValueError("dense_gemv takes binary16 or bfloat16 x and weight of one dtype")
    if bias is not None and bias.dtype != x.dtype:
        raise ValueError("bias must have x's dtype")
    if weight.dim() != 2 or weight.stride(-1) != 1:
        raise ValueError("weight must be a row-major [N, K] matrix")
    k = x.shape[-1]
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError(f"x has {k} columns, weight {weight.shape[1]}")
    rows = x.reshape(-1, k)
    m = rows.shape[0]
    ld = rows.stride(0) if m > 1 else k
    if rows.stride(-1) != 1 or ld < k or ld % 8 or rows.data_ptr() % 16:
        rows = rows.contiguous()
        ld = k
    if m > MAX_ROWS:
        raise ValueError(f"dense_gemv takes at most {MAX_ROWS} rows (got {m}); "
                         "larger batches are a GEMM")
    y = torch.empty(m, n, device=device, dtype=x.dtype)
    if m and n:
        b = bias.contiguous() if bias is not None else None
        _lib.check(_lib.load().w8a8_dense_gemv(
            rows.data_ptr(), ld, weight.data_ptr(),
            weight.stride(0), b.data_ptr() if b is not None else None, y.data_ptr(), n,
            _lib.dtype_code(x.dtype), m, n, k, _lib.stream_handle(device)), "w8a8_dense_gemv")
    return y.view(*x.shape[:-1], n)


class DecodeLMHead(nn.Module):
    """The model's ``lm_head`` with decode batches on ``dense_gemv``.

    Holds the wrapped module (its weight is used in place, not copied).
    GPU tensors only.  Up to 16 rows with supported operands run the kernel;
    larger batches (and shapes outside the kernel's range) take the module's
    own GEMM on the GPU (the reference's ``F.linear``).
    """

    def __init__(self, linear: nn.Linear) -> None:
        super().__init__()
        self.linear = linear

    @property
    def weight(self) -> torch.Tensor:
        return self.linear.weight

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        bias = getattr(self.linear, "bias", None)
        _lib.require_cuda(hidden, self.linear.weight, bias)
        if dense_gemv_supported(hidden, self.linear.weight, bias):
            return dense_gemv(hidden, self.linear.weight, bias)
        return F.linear(hidden, self.linear.weight, bias)
