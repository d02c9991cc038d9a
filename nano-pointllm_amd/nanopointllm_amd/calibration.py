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

# Modules whose inputs carry their channels on dimension 1 (N, C, ...); every
# other module reads its channels from the last dimension.
_CHANNEL_FIRST = (nn.Conv1d, nn.Conv2d)


def _channel_dim(module: nn.Module) -> int:
    return 1 if isinstance(module, _CHANNEL_FIRST) else -1


def _channel_rows(values: torch.Tensor, dim: int) -> torch.Tensor:
    """``values`` as a 2-D [samples, channels] view, channels from ``dim``."""
    return values.movedim(dim, -1).reshape(-1, values.shape[dim])


class ActivationAbsmaxCollector(AbstractContextManager):
    """Collect tensor and input-channel ranges without changing model outputs
    (w8a8.py:265-314; same attributes and ``static_scales()``).

    The running maxima stay on the inputs' device and each hook updates them
    in place, so a calibration forward never waits for the host.  The tensor
    maximum is the maximum of the channel maxima, so one running vector per
    module is kept (a running scalar for 0-d inputs); ``tensor_absmax`` and
    ``channel_absmax`` copy them to the host when they are read.
    """

    def __init__(self, modules: dict[str, nn.Module]) -> None:
        self.modules = modules
        self.samples: dict[str, int] = defaultdict(int)
        self._channel_peaks: dict[str, torch.Tensor] = {}  # f32 [channels]
        self._scalar_peaks: dict[str, torch.Tensor] = {}   # f32 [], 0-d inputs
        self._handles = []

    def __enter__(self) -> "ActivationAbsmaxCollector":
        self._handles = [module.register_forward_pre_hook(self._observer(name, module))
                         for name, module in self.modules.items()]
        return self

    def __exit__(self, exc_type, exc_value, traceback) -> None:
        while self._handles:
            self._handles.pop().remove()

    def _observer(self, name: str, module: nn.Module):
        dim = _channel_dim(module)

        def observe(_module, inputs) -> None:
            if not inputs or not isinstance(inputs[0], torch.Tensor):
                raise TypeError(f"{name} does not have a tensor first input")
            values = inputs[0].detach()
            if values.dim() == 0:
                store, peak = self._scalar_peaks, values.abs().float()
            else:
                store = self._channel_peaks
                peak = _channel_rows(values, dim).abs().amax(dim=0).float()
                self.samples[name] += values.numel() // values.shape[dim]
            held = store.get(name)
            if held is None:
                store[name] = peak
            else:
                torch.maximum(held, peak, out=held)
        return observe

    def _module_peaks(self) -> dict[str, torch.Tensor]:
        """One 0-d device tensor per observed module: its tensor-wide absmax."""
        peaks: dict[str, torch.Tensor] = {}
        for store in (self._channel_peaks, self._scalar_peaks):
            for name, held in store.items():
                top = held.amax()
                peaks[name] = top if name not in peaks else torch.maximum(peaks[name], top)
        return peaks

    @property
    def tensor_absmax(self) -> dict[str, float]:
        peaks = self._module_peaks()
        if not peaks:
            return defaultdict(float)
        host = torch.stack(list(peaks.values())).cpu().tolist()
        return defaultdict(float, zip(peaks, host))

    @property
    def channel_absmax(self) -> dict[str, torch.Tensor]:
        return {name: held.cpu() for name, held in self._channel_peaks.items()}

    def static_scales(self) -> dict[str, torch.Tensor]:
        peaks = self._module_peaks()
        missing = sorted(set(self.modules) - set(peaks))
        if missing:
            raise RuntimeError(f"no activation calibration for modules: {missing[:3]}")
        # Every module's static scale (scale_from_absmax, w8a8.py:46-50,
        # 94-98) in one device computation and one copy to the host.
        scales = _w.scale_from_absmax(torch.stack(list(peaks.values()))).cpu()
        return {name: scales[i] for i, name in enumerate(peaks)}


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
        self._handles = [module.register_forward_pre_hook(self._hook(name))
                         for name, module in self.modules.items()]
        return self

    def __exit__(self, exc_type, exc_value, traceback) -> None:
        while self._handles:
            self._handles.pop().remove()

    def _hook(self, name: str):
        def quantize(module, inputs):
            smoothing = self.input_smoothing_scales.get(name)
            # Static mode needs a calibrated scale for every module (a missing
            # one raises KeyError, as the reference's lookup does).
            static = self.static_scales[name] if self.mode == "static" else None
            return (_qdq_input(inputs[0], _channel_dim(module), smoothing, static), *inputs[1:])
        return quantize


def _qdq_input(values: torch.Tensor, dim: int, smoothing: torch.Tensor | None,
               static: torch.Tensor | None) -> torch.Tensor:
    """``values / smoothing`` then static or per-token QDQ along channel ``dim``.

    16-bit rows with channels last take the fused prologue kernel (divide and
    quantization in one pass); other inputs divide in torch and quantize with
    the GPU quantizers of the same contract."""
    if smoothing is not None:
        smoothing = smoothing.to(device=values.device)   # calibration keeps it on the CPU
    if dim == -1 and values.dtype in (torch.float16, torch.bfloat16):
        out = _w.prologue_quant(values, smooth=smoothing,
                                static_scale=None if static is None else float(static))
        scale = out.scale if static is not None else out.scale.unsqueeze(-1)
        return (out.q.float() * scale).to(values.dtype)
    if smoothing is not None:
        shape = [1] * values.dim()
        shape[dim] = smoothing.numel()
        values = values / smoothing.to(values.dtype).reshape(shape)
    if static is not None:
        return _w.static_activation_qdq(values, static.to(values.device))
    return _w.dynamic_per_token_activation_qdq(values, axis=dim)[0]


def _weight_qdq(granularity: str, group_size: int):
    if granularity == "per_output":
        return _w.per_output_weight_qdq
    if granularity == "group":
        return lambda weight: _w.groupwise_weight_qdq(weight, group_size=group_size)
    raise ValueError("weight granularity must be per_output or group")


@torch.no_grad()
def apply_weight_qdq(modules: dict[str, nn.Module], *, granularity: str,
                     group_size: int = 128) -> dict[str, dict[str, Any]]:
    """Fake-quantize module weights in place (w8a8.py:417-447), with the
    reference's report per module.  Each module's integer range and error are
    reduced on the device and reach the host in one copy."""
    qdq = _weight_qdq(granularity, group_size)
    reports = {}
    for name, module in modules.items():
        weight = getattr(module, "weight", None)
        if weight is None:
            raise TypeError(f"{name} has no weight")
        dequantized, quantized, scales = qdq(weight)
        rmse = (dequantized.float() - weight.detach().float()).square().mean().sqrt()
        q_lo, q_hi, err = torch.stack([quantized.min().double(), quantized.max().double(),
                                       rmse.double()]).tolist()
        shape = list(weight.shape)
        weight.copy_(dequantized)
        reports[name] = {
            "shape": shape,
            "parameters": weight.numel(),
            "granularity": granularity,
            "group_size": group_size if granularity == "group" else None,
            "scale_shape": list(scales.shape),
            "quantized_min": int(q_lo),
            "quantized_max": int(q_hi),
            "rmse": err,
        }
    return reports


_SMOOTH_EPS = 1e-5


def _smoothing_vector(act_absmax: torch.Tensor, weight_absmax: torch.Tensor,
                      alpha: float) -> torch.Tensor:
    """SmoothQuant's per-channel factor (w8a8.py:399-404): ``max(a^alpha /
    w^(1-alpha), 1e-5)`` with both maxima floored at 1e-5, then stored as
    binary16 and floored again."""
    ratio = act_absmax.clamp_min(_SMOOTH_EPS).pow(alpha) / \
        weight_absmax.clamp_min(_SMOOTH_EPS).pow(1.0 - alpha)
    return ratio.clamp_min(_SMOOTH_EPS).to(torch.float16).float().clamp_min(_SMOOTH_EPS)


@torch.no_grad()
def apply_smoothquant_transform(modules: dict[str, nn.Module],
                                channel_absmax: dict[str, torch.Tensor], *,
                                alpha: float = 0.5
                                ) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    """Exact ``x/s, W*s`` smoothing and the post-transform static A8 scales
    (w8a8.py:370-414).  Each weight is scaled in place along its input
    channels (dimension 1); the smoothed activation maxima of all modules are
    converted to static scales together on the device.  Returns
    ``(input_smoothing_scales, activation_scales)`` on the CPU like the
    reference."""
    if not 0.0 <= alpha <= 1.0:
        raise ValueError("SmoothQuant alpha must be in [0, 1]")
    missing = sorted(set(modules) - set(channel_absmax))
    if missing:
        raise RuntimeError(f"no channel calibration for modules: {missing[:3]}")
    vectors: dict[str, torch.Tensor] = {}
    post_peaks: list[torch.Tensor] = []
    for name, module in modules.items():
        weight = module.weight
        channels = weight.shape[1]
        # Per input channel |W| max: input channels last, everything else rows.
        weight_absmax = _channel_rows(weight.detach().float(), 1).abs().amax(dim=0)
        act_absmax = channel_absmax[name].float().to(weight.device)
        if act_absmax.numel() != weight_absmax.numel():
            raise ValueError(f"activation/weight channel mismatch for {name}: "
                             f"{act_absmax.numel()} versus {weight_absmax.numel()}")
        smoothing = _smoothing_vector(act_absmax, weight_absmax, alpha)
        shape = [1] * weight.dim()
        shape[1] = channels
        weight.mul_(smoothing.to(weight.dtype).reshape(shape))
        vectors[name] = smoothing
        post_peaks.append((act_absmax / smoothing).amax())
    if not vectors:
        return {}, {}
    device = post_peaks[0].device
    scales = _w.scale_from_absmax(torch.stack([p.to(device) for p in post_peaks])).cpu()
    input_scales = {name: v.cpu() for name, v in vectors.items()}
    activation_scales = {name: scales[i] for i, name in enumerate(vectors)}
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
    # The 16-bit h must reach each down projection through its module call
    # (the hooked path): no static scale, no two-phase int8 h.
    saved = {idx: (m.h_scale, m.two_phase) for idx, m in mlps.items()}
    for m in mlps.values():
        m.h_scale, m.two_phase = None, False
    try:
        with ActivationAbsmaxCollector({str(i): m.down for i, m in mlps.items()}) as col:
            run()
    finally:
        for idx, m in mlps.items():
            m.h_scale, m.two_phase = saved[idx]
    return {int(name): float(scale) for name, scale in col.static_scales().items()}
