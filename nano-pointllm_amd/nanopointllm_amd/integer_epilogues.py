"""Integer output contracts of the hardware model, on the GPU.

* a17 - INT32 -> A8 requantization with an unsigned multiplier and a
  round-to-nearest-even right shift
  (architecture_simulator/gtsu_cycle/requant.py:62-119): the scale compiler
  runs on the host (it is scalar pack-time work, in the reference's own float
  arithmetic); ``requantize_int32`` and the fused int8-in linear run in HIP.
* a18 - INT32 x FP16 x FP16 -> BF16 with one rounding of the exact product
  (architecture_simulator/gtsu_cycle/bf16_dequant.py:47-77): elementwise over
  caller accumulators, or fused as the ``EPI_DEQUANT_BF16_EXACT`` epilogue of
  ``w8a8.linear_dynamic`` / ``w8a8.linear_i8in``.

Multipliers are uint32 values; torch has no general uint32 arithmetic, so they
travel as int32 tensors holding the same bit patterns.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn

from . import _lib, w8a8

_UINT32_MAX = (1 << 32) - 1


def _fp16(value: float) -> float:
    """Round to binary16 and back, as the reference does (requant.py:192-193)."""
    return struct.unpack("e", struct.pack("e", value))[0]


@dataclass(frozen=True)
class CompiledRequantScale:
    """Same fields as the reference's compiled scale (requant.py:49-59)."""

    activation_scale: float
    weight_scale: float
    output_scale: float
    exact_ratio: float
    multiplier: int
    right_shift: int
    represented_ratio: float
    relative_error: float


def compile_requant_ratio(ratio: float) -> tuple[int, int]:
    """``compile_requant_ratio`` (requant.py:80-95): the largest right shift
    (<= 63) whose rounded multiplier fits uint32."""
    if ratio <= 0 or not math.isfinite(ratio):
        raise ValueError("requant ratio must be positive and finite")
    shift = min(63, math.floor(math.log2(_UINT32_MAX / ratio)))
    if shift < 0:
        raise OverflowError("requant ratio exceeds UINT32 multiplier range")
    mult = round(ratio * (1 << shift))
    if mult > _UINT32_MAX:
        shift -= 1
        mult = round(ratio * (1 << shift))
    if mult <= 0 or shift < 0:
        raise OverflowError("requant ratio is outside multiplier/shift range")
    return mult, shift


def compile_fp16_requant_scale(activation_scale: float, weight_scale: float,
                               output_scale: float) -> CompiledRequantScale:
    """``compile_fp16_requant_scale`` (requant.py:62-77)."""
    a, w, o = _fp16(activation_scale), _fp16(weight_scale), _fp16(output_scale)
    if min(a, w, o) <= 0 or not all(math.isfinite(t) for t in (a, w, o)):
        raise ValueError("requant scales must be positive finite FP16 values")
    ratio = a * w / o
    mult, shift = compile_requant_ratio(ratio)
    represented = mult / (1 << shift)
    return CompiledRequantScale(a, w, o, ratio, mult, shift, represented,
                                abs(represented - ratio) / ratio)


def compile_per_output(activation_scale: float, weight_scales, output_scale: float,
                       device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output ``(multiplier, right_shift)`` device tensors (int32 holding
    uint32 multipliers, int32 shifts) for one static activation scale, the
    per-output weight scales and one output scale."""
    ws = np.asarray(torch.as_tensor(weight_scales).detach().float().cpu().numpy(), np.float64)
    mult = np.empty(ws.size, np.uint32)
    shift = np.empty(ws.size, np.int32)
    for i, w in enumerate(ws.reshape(-1)):
        c = compile_fp16_requant_scale(activation_scale, float(w), output_scale)
        mult[i], shift[i] = c.multiplier, c.right_shift
    return (torch.from_numpy(mult.view(np.int32)).to(device),
            torch.from_numpy(shift).to(device))


def _as_i32(t: torch.Tensor | None, n: int, name: str) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.int32 or t.numel() != n:
        raise ValueError(f"{name} must be an int32 tensor of {n} values")
    return t.contiguous()


def requantize_int32(acc: torch.Tensor, bias: torch.Tensor | None, multiplier: torch.Tensor,
                     right_shift: torch.Tensor) -> torch.Tensor:
    """``requantize_int32`` (requant.py:98-119) for int32 ``acc[..., N]`` with
    per-column ``bias`` (int32, nullable), ``multiplier`` (uint32 bits in
    int32) and ``right_shift`` (int32, 0..63).  Returns int8."""
    device = _lib.require_cuda(acc, bias, multiplier, right_shift)
    if acc.dtype != torch.int32:
        raise ValueError("accumulators must be int32")
    a2, lda = w8a8._rows_view(acc)
    m, n = a2.shape
    mult = _as_i32(multiplier, n, "multiplier")
    shift = _as_i32(right_shift, n, "right_shift")
    b = _as_i32(bias, n, "bias")
    y = torch.empty((m, n), dtype=torch.int8, device=device)
    if m and n:
        _lib.check(_lib.load().w8a8_requantize_i32(
            a2.data_ptr(), lda, _lib.ptr(b), mult.data_ptr(), shift.data_ptr(), y.data_ptr(), n,
            m, n, _lib.stream_handle(device)), "w8a8_requantize_i32")
    return y.reshape(acc.shape)


def _f16_bits(scales: torch.Tensor) -> torch.Tensor:
    """Binary16 bit patterns of scales given as float16 / float32 values."""
    return scales.detach().to(torch.float16).contiguous().view(torch.int16)


def dequantize_int32_to_bf16(acc: torch.Tensor, activation_scale: torch.Tensor,
                             weight_scale: torch.Tensor) -> torch.Tensor:
    """``dequantize_int32_to_bf16`` (bf16_dequant.py:47-77) for int32
    ``acc[M, N]``: ``activation_scale`` per row ([M] or one value) and
    ``weight_scale`` per column ([N]), as binary16 values (float16 tensors, or
    int16 tensors holding the bit patterns).  Returns bfloat16 [M, N]."""
    device = _lib.require_cuda(acc, activation_scale, weight_scale)
    if acc.dtype != torch.int32:
        raise ValueError("accumulators must be int32")
    a2, lda = w8a8._rows_view(acc)
    m, n = a2.shape
    sa = activation_scale if activation_scale.dtype == torch.int16 else _f16_bits(activation_scale)
    sw = weight_scale if weight_scale.dtype == torch.int16 else _f16_bits(weight_scale)
    sa = sa.reshape(-1)
    if sa.numel() == 1 and m != 1:
        sa = sa.expand(m)
    sa, sw = sa.contiguous(), sw.reshape(-1).contiguous()
    if sa.numel() != m or sw.numel() != n:
        raise ValueError("scales must be one per row and one per column")
    y = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    if m and n:
        _lib.check(_lib.load().w8a8_dequant_i32_bf16(
            a2.data_ptr(), lda, sa.data_ptr(), sw.data_ptr(), y.data_ptr(), n, m, n,
            _lib.stream_handle(device)), "w8a8_dequant_i32_bf16")
    return y.reshape(acc.shape)


def linear_i8in_requant(xq: torch.Tensor, w_packed: torch.Tensor, multiplier: torch.Tensor,
                        right_shift: torch.Tensor, bias: torch.Tensor | None, n: int, *,
                        in_features: int | None = None) -> torch.Tensor:
    """Static-A8 linear with the integer requantization fused into the
    product's epilogue: int8 ``requantize_int32(xq @ wq^T, bias, multiplier,
    right_shift)``."""
    device = _lib.require_cuda(xq, w_packed, multiplier, right_shift, bias)
    if xq.dtype != torch.int8:
        raise ValueError("activations must be int8")
    x2, ldq = w8a8._rows_view(xq)
    m, k = x2.shape
    w8a8._check_operands(k, w_packed, None, None, n, in_features)
    mult = _as_i32(multiplier, n, "multiplier")
    shift = _as_i32(right_shift, n, "right_shift")
    b = _as_i32(bias, n, "bias")
    y = torch.empty((m, n), dtype=torch.int8, device=device)
    if m and n:
        ws = w8a8._workspace(m, k, device)
        _lib.check(_lib.load().w8a8_linear_i8in_requant(
            x2.data_ptr(), ldq, w_packed.data_ptr(), mult.data_ptr(), shift.data_ptr(),
            _lib.ptr(b), y.data_ptr(), n, m, n, k, ws.data_ptr(), ws.numel(),
            _lib.stream_handle(device)), "w8a8_linear_i8in_requant")
    return y.reshape(*xq.shape[:-1], n)


class StaticA8RequantLinear(nn.Module):
    """int8 in -> int8 out linear of the static-A8 requant mode.

    Weights are quantized per output row (per_output_weight_qdq,
    nanopointllm/compression/w8a8.py:53-62) and packed once; the per-output
    multiplier / right shift come from ``compile_fp16_requant_scale`` of the
    calibrated activation scale, each weight scale and the output scale.
    ``bias_i32`` (optional) is in accumulator units, added before the
    multiplier as in the hardware model.
    """

    def __init__(self, linear: nn.Linear, activation_scale: float, output_scale: float,
                 bias_i32: torch.Tensor | None = None):
        super().__init__()
        weight = linear.weight.detach()
        _lib.require_cuda(weight)
        _, q, s = w8a8.per_output_weight_qdq(weight.float())
        self.out_features, self.in_features = q.shape
        self.register_buffer("packed", w8a8.pack_rows(q))
        self.register_buffer("weight_scale", s)
        mult, shift = compile_per_output(activation_scale, s, output_scale, weight.device)
        self.register_buffer("multiplier", mult)
        self.register_buffer("right_shift", shift)
        self.register_buffer("bias_i32", None if bias_i32 is None else
                             _as_i32(bias_i32.to(weight.device), self.out_features, "bias_i32"))
        self.activation_scale = float(activation_scale)
        self.output_scale = float(output_scale)

    def forward(self, xq: torch.Tensor) -> torch.Tensor:
        return linear_i8in_requant(xq, self.packed, self.multiplier, self.right_shift,
                                   self.bias_i32, self.out_features,
                                   in_features=self.in_features)
