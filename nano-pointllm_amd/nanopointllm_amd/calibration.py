"""Calibration and fake-quant API for the W8A8 path (nanopointllm/compression/
w8a8.py:265-447), on the GPU.

The reference calibrates through ``nn.Module`` forward pre-hooks, which never
fire on its packed decode paths (they call ``F.linear`` on packed copies).
Here every packed call site goes through a module call (``W8A8MLP.down``,
``W8A8PackedQKV.linear``, ...), so the same hook-based API works on the W8A8
modules, and :func:`calibrate_h_scales` returns the static scales of the int8
MLP chain (``inject_w8a8(h_scales=...)``).

* :class:`ActivationAbsmaxCollector` - per-module tensor and input-channel
  absmax (w8a8.py:265-314), same attributes and ``static_scales()``.
* :class:`SequentialActivationQDQ` - activation QDQ injected at module inputs,
  static or per-token dynamic, with optional SmoothQuant input smoothing
  (w8a8.py:317-367); the divide and quantization run in the fused prologue.
* :func:`apply_weight_qdq` - per-output or groupwise weight fake-quant with the
  reference's report (w8a8.py:417-447).
* :func:`apply_smoothquant_transform` - exact ``x/s, W*s`` smoothing and the
  post-transform static scales (w8a8.py:370-414).
* :func:`smoothquant_hardware_report` - storage and foldability of the
  smoothing vectors (w8a8.py:217-251).
"""
from __future__ import annotations

from collections import defaultdict
from contextlib import AbstractContextManager
from typing import Any, Callable

import torch
import torch.nn as nn

from . import w8a8 as _w

_CONV = (nn.Conv1d, nn.Conv2d)


class ActivationAbsmaxCollector(AbstractContextManager):
    """Collect tensor and input-channel ranges without changing model outputs
    (w8a8.py:265-314)."""

    def __init__(self, modules: dict[str, nn.Module]) -> None:
        self.modules = modules
        self.tensor_absmax: dict[str, float] = defaultdict(float)
        self.channel_absmax: dict[str, torch.Tensor] = {}
        self.samples: dict[str, int] = defaultdict(int)
        self._handles = []
        self._device = torch.device("cuda")

    def __enter__(self) -> "ActivationAbsmaxCollector":
        for name, module in self.modules.items():
            self._handles.append(module.register_forward_pre_hook(self._hook(name)))
        return self

    def __exit__(self, exc_type, exc_value, traceback) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles.clear()

    def _hook(self, name: str):
        def collect(module, inputs) -> None:
            if not inputs or not isinstance(inputs[0], torch.Tensor):
                raise TypeError(f"{name} does not have a tensor first input")
            values = inputs[0].detach().float()
            self._device = values.device
            self.tensor_absmax[name] = max(self.tensor_absmax[name],
                                           float(values.abs().max().item()))
            if values.dim() >= 1:
                if isinstance(module, _CONV):
                    dims = tuple(i for i in range(values.dim()) if i != 1)
                    flat = values.abs().amax(dim=dims).cpu()
                    channels = values.shape[1]
                else:
                    flat = values.reshape(-1, values.shape[-1]).abs().amax(dim=0).cpu()
                    channels = values.shape[-1]
                previous = self.channel_absmax.get(name)
                self.channel_absmax[name] = flat if previous is None else torch.maximum(previous,
                                                                                        flat)
                self.samples[name] += values.numel() // channels
        return collect

    def static_scales(self) -> dict[str, torch.Tensor]:
        missing = sorted(set(self.modules) - set(self.tensor_absmax))
        if missing:
            raise RuntimeError(f"no activation calibration for modules: {missing[:3]}")
        return {name: _w.static_activation_scale(absmax, device=self._device).cpu()
                for name, absmax in self.tensor_absmax.items()}


class SequentialActivationQDQ(AbstractContextManager):
    """Inject activation QDQ at every selected module input (w8a8.py:317-367).

    Linear inputs of binary16 / bfloat16 go through the fused prologue kernel
    (smoothing divide + quantization); other inputs (binary32 rows, conv
    channels) use the GPU quantization of the same contract.
    """

    def __init__(self, modules: dict[str, nn.Module], *, mode: str,
                 static_scales: dict[str, torch.Tensor] | None = None,
                 input_smoothing_scales: dict[str, torch.Tensor] | None = None) -> None:
        if mode not in ("static", "dynamic_per_token"):
            raise ValueError("activation mode must be static or dynamic_per_token")
        if mode == "static" and static_scales is None:
            raise ValueError("static activation mode requires calibrated scales")
        self.modules = modules
        self.mode = mode
        self.static_scales = static_scales or {}
        self.input_smoothing_scales = input_smoothing_scales or {}
        self._handles = []

    def __enter__(self) -> "SequentialActivationQDQ":
        for name, module in self.modules.items():
            self._handles.append(module.register_forward_pre_hook(self._hook(name)))
        return self

    def __exit__(self, exc_type, exc_value, traceback) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles.clear()

    def _hook(self, name: str):
        def quantize(module, inputs):
            values = inputs[0]
            smoothing = self.input_smoothing_scales.get(name)
            static = self.static_scales.get(name) if self.mode == "static" else None
            conv = isinstance(module, _CONV)
            if not conv and values.dtype in (torch.float16, torch.bfloat16):
                replacement = _fused_qdq(values, smoothing, static)
            else:
                if smoothing is not None:
                    sm = smoothing.to(device=values.device, dtype=values.dtype)
                    if conv:
                        shape = [1] * values.dim()
                        shape[1] = sm.numel()
                        sm = sm.reshape(shape)
                    values = values / sm
                if static is not None:
                    replacement = _w.static_activation_qdq(values, static.to(values.device))
                else:
                    replacement, _ = _w.dynamic_per_token_activation_qdq(
                        values, axis=1 if conv else -1)
            return (replacement, *inputs[1:])
        return quantize


def _fused_qdq(values: torch.Tensor, smoothing: torch.Tensor | None,
               static: torch.Tensor | None) -> torch.Tensor:
    if smoothing is not None:
        smoothing = smoothing.to(device=values.device)   # calibration keeps it on the CPU
    out = _w.prologue_quant(values, smooth=smoothing,
                            static_scale=None if static is None else float(static))
    s = out.scale if static is not None else out.scale.unsqueeze(-1)
    return (out.q.float() * s).to(values.dtype)


@torch.no_grad()
def apply_weight_qdq(modules: dict[str, nn.Module], *, granularity: str,
                     group_size: int = 128) -> dict[str, dict[str, Any]]:
    """Fake-quantize module weights in place (w8a8.py:417-447)."""
    if granularity not in ("per_output", "group"):
        raise ValueError("weight granularity must be per_output or group")
    reports = {}
    for name, module in modules.items():
        if not hasattr(module, "weight"):
            raise TypeError(f"{name} has no weight")
        weight = module.weight
        if granularity == "per_output":
            dequantized, quantized, scales = _w.per_output_weight_qdq(weight)
        else:
            dequantized, quantized, scales = _w.groupwise_weight_qdq(weight, group_size=group_size)
        error = dequantized.float() - weight.detach().float()
        module.weight.copy_(dequantized)
        reports[name] = {
            "shape": list(weight.shape),
            "parameters": weight.numel(),
            "granularity": granularity,
            "group_size": group_size if granularity == "group" else None,
            "scale_shape": list(scales.shape),
            "quantized_min": int(quantized.min().item()),
            "quantized_max": int(quantized.max().item()),
            "rmse": float(error.square().mean().sqrt().item()),
        }
    return reports


@torch.no_grad()
def apply_smoothquant_transform(modules: dict[str, nn.Module],
                                channel_absmax: dict[str, torch.Tensor], *,
                                alpha: float = 0.5
                                ) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    """Exact ``x/s, W*s`` smoothing and the post-transform static A8 scales
    (w8a8.py:370-414): ``s = max(a^alpha / w^(1-alpha), 1e-5)`` per input
    channel, stored as binary16 (clamped again at 1e-5), the weight scaled in
    place.  Returns ``(input_smoothing_scales, activation_scales)`` on the CPU
    like the reference."""
    if not 0.0 <= alpha <= 1.0:
        raise ValueError("SmoothQuant alpha must be in [0, 1]")
    missing = sorted(set(modules) - set(channel_absmax))
    if missing:
        raise RuntimeError(f"no channel calibration for modules: {missing[:3]}")
    input_scales, activation_scales = {}, {}
    eps = 1e-5
    for name, module in modules.items():
        weight = module.weight.detach().float()
        if isinstance(module, _CONV):
            weight_absmax = weight.abs().amax(dim=tuple(i for i in range(weight.dim()) if i != 1))
            shape = [1] * weight.dim()
            shape[1] = weight.shape[1]
        else:
            weight_absmax = weight.reshape(weight.shape[0], -1).abs().amax(dim=0)
            shape = [1, weight.shape[1]]
        act_absmax = channel_absmax[name].float().to(weight.device)
        if act_absmax.numel() != weight_absmax.numel():
            raise ValueError(f"activation/weight channel mismatch for {name}: "
                             f"{act_absmax.numel()} versus {weight_absmax.numel()}")
        smoothing = (act_absmax.clamp_min(eps).pow(alpha)
                     / weight_absmax.clamp_min(eps).pow(1.0 - alpha)).clamp_min(eps)
        smoothing = smoothing.to(torch.float16).float().clamp_min(eps)
        module.weight.mul_(smoothing.to(module.weight.dtype).reshape(shape))
        post_absmax = (act_absmax / smoothing).amax()
        input_scales[name] = smoothing.cpu()
        activation_scales[name] = _w.static_activation_scale(post_absmax,
                                                             device=weight.device).cpu()
    return input_scales, activation_scales


_SHARED_INPUT_STATUS = (
    (("q_proj", "k_proj", "v_proj"), "not_foldable_independently_shared_qkv_input"),
    (("gate_proj", "up_proj"), "not_foldable_independently_shared_gate_up_input"),
)


def smoothquant_hardware_report(modules: dict[str, nn.Module],
                                input_smoothing_scales: dict[str, torch.Tensor]
                                ) -> dict[str, Any]:
    """Storage and foldability of independent per-module smoothing vectors
    (w8a8.py:217-251), in the reference's report format.

    Q/K/V and gate/up read one shared producer output, so a vector per module
    cannot be folded into that producer; any other module needs its producer's
    fan-out and residual path checked first.  Every vector is stored as
    binary16 and divided at run time (here inside the activation prologue)."""
    rows: dict[str, dict[str, Any]] = {}
    total = 0
    for name, module in modules.items():
        channels = int(input_smoothing_scales[name].numel())
        total += channels
        status = next((s for parts, s in _SHARED_INPUT_STATUS if any(p in name for p in parts)),
                      "requires_producer_fanout_and_residual_proof")
        rows[name] = {
            "channels": channels,
            "storage_bytes_fp16": channels * 2,
            "current_runtime_channelwise_divide": True,
            "offline_fold_status": status,
            "module_type": type(module).__name__,
        }
    return {
        "scheme": "independent_per_module_smoothing_vectors",
        "vector_count": len(rows),
        "total_scale_values": total,
        "total_storage_bytes_fp16": total * 2,
        "runtime_overhead_zero": False,
        "reason": ("independent Q/K/V and Gate/Up vectors cannot all fold into their "
                   "single shared producer; joint-group smoothing is required"),
        "modules": rows,
    }


def calibrate_h_scales(model: nn.Module, run: Callable[[], Any]) -> dict[int, float]:
    """Static scales for the int8 MLP chain: runs ``run()`` (calibration
    forwards) with every injected ``W8A8MLP`` keeping ``h`` in 16 bits,
    collects the absmax of each down projection's input, and returns
    ``{layer index: static_activation_scale(absmax)}`` for
    ``inject_w8a8(model, h_scales=...)`` or ``W8A8MLP.h_scale``."""
    from .linear import W8A8MLP

    mlps = {idx: layer.mlp.w8a8_mlp for idx, layer in enumerate(model.model.layers)
            if isinstance(getattr(getattr(layer, "mlp", None), "w8a8_mlp", None), W8A8MLP)}
    if not mlps:
        raise RuntimeError("no injected W8A8 MLPs to calibrate")
    saved = {idx: m.h_scale for idx, m in mlps.items()}
    for m in mlps.values():
        m.h_scale = None
    try:
        with ActivationAbsmaxCollector({str(i): m.down for i, m in mlps.items()}) as col:
            run()
    finally:
        for idx, m in mlps.items():
            m.h_scale = saved[idx]
    return {int(name): float(scale) for name, scale in col.static_scales().items()}
