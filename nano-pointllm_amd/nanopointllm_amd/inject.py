"""Install the W8A8 linears into a LLaMA-style model.

Modelled on ``inject_paged_attention`` (nanopointllm/llama/inject_paged.py:11-33):
walk ``model.model.layers`` and replace, in place, the dense projections of
each decoder layer.

* Module call sites - ``self.q_proj(x)`` ... ``self.o_proj(out)`` in the
  prefill / mixed path (llama/paged_attention.py:1349-1352, 1376, 1488) and
  ``self.gate_proj(x)`` / ``self.up_proj(x)`` / ``self.down_proj(h)`` in the
  unpacked MLP branch (llama/lightweight_runner.py:389-404) - keep working
  unchanged because every ``nn.Linear`` becomes a :class:`W8A8Linear` with the
  same ``forward(x) -> y`` contract.
* Packed call sites - ``F.linear(staged, packed_qkv_weight, b)``
  (paged_attention.py:97-115, 283-305) and the packed gate/up -> SiLU*mul ->
  down branch (lightweight_runner.py:320-383) - get the packed modules
  attached as ``self_attn.w8a8_qkv`` and ``mlp.w8a8_mlp``, and the helpers
  below mirror the reference helpers' signatures and return shapes.

All weights are quantized per output row (per_output_weight_qdq,
nanopointllm/compression/w8a8.py:53-62) on the GPU and packed once.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .linear import W8A8GateUpSiluMul, W8A8Linear, W8A8MLP, W8A8PackedQKV, _rows2

_ATTN_LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj")
_MLP_LINEARS = ("gate_proj", "up_proj", "down_proj")


def _attn_geometry(attn: nn.Module, q_proj: nn.Module) -> tuple[int, int, int]:
    cfg = getattr(attn, "config", None)
    heads = getattr(attn, "num_heads", None) or getattr(cfg, "num_attention_heads", None)
    kv_heads = (getattr(attn, "num_kv_heads", None) or getattr(attn, "num_key_value_heads", None)
                or getattr(cfg, "num_key_value_heads", None) or heads)
    head_dim = getattr(attn, "head_dim", None)
    if heads is None:
        raise ValueError("attention module does not expose its head count")
    if head_dim is None:
        head_dim = q_proj.out_features // heads
    return int(heads), int(kv_heads), int(head_dim)


def inject_w8a8(hf_model: nn.Module, *, h_scales: dict[int, float] | None = None,
                pack: bool = True, weight_cache=None, verify_source: bool = False
                ) -> dict[str, int]:
    """Replace the decoder layers' projections with W8A8 modules (in place).

    ``h_scales`` optionally maps a layer index to a calibrated static scale for
    the SiLU*mul output, which turns that layer's packed MLP into the int8
    chain (gate/up writes int8, down consumes it).  ``weight_cache`` is a
    directory of pre-quantized, pre-packed weights (``weight_cache.py``):
    entries present are loaded (checksummed; ``verify_source`` also checks
    them against the model's weights), missing ones are built and stored.
    Returns counts of replaced modules.  The model's weights must live on the
    GPU.
    """
    layers = hf_model.model.layers
    counts = {"linear": 0, "packed_qkv": 0, "packed_mlp": 0}
    for idx, layer in enumerate(layers):
        attn = getattr(layer, "self_attn", None)
        mlp = getattr(layer, "mlp", None)
        if attn is not None and all(hasattr(attn, n) for n in _ATTN_LINEARS):
            q, k, v = attn.q_proj, attn.k_proj, attn.v_proj
            prefix = f"layers.{idx}.self_attn."
            cache = dict(weight_cache=weight_cache, verify_source=verify_source)
            if pack and not isinstance(q, W8A8Linear):
                heads, kv_heads, head_dim = _attn_geometry(attn, q)
                attn.w8a8_qkv = W8A8PackedQKV(q, k, v, num_heads=heads, num_kv_heads=kv_heads,
                                              head_dim=head_dim, cache_key=prefix + "packed_qkv",
                                              **cache)
                counts["packed_qkv"] += 1
            for name in _ATTN_LINEARS:
                mod = getattr(attn, name)
                if not isinstance(mod, W8A8Linear):
                    setattr(attn, name, W8A8Linear.from_linear(mod, cache_key=prefix + name,
                                                               **cache))
                    counts["linear"] += 1
        if mlp is not None and all(hasattr(mlp, n) for n in _MLP_LINEARS):
            g, u, d = mlp.gate_proj, mlp.up_proj, mlp.down_proj
            prefix = f"layers.{idx}.mlp."
            cache = dict(weight_cache=weight_cache, verify_source=verify_source)
            if pack and not isinstance(g, W8A8Linear):
                scale = None if h_scales is None else h_scales.get(idx)
                mlp.w8a8_mlp = W8A8MLP(g, u, d, h_scale=scale, cache_prefix=prefix, **cache)
                counts["packed_mlp"] += 1
            for name in _MLP_LINEARS:
                mod = getattr(mlp, name)
                if not isinstance(mod, W8A8Linear):
                    setattr(mlp, name, W8A8Linear.from_linear(mod, cache_key=prefix + name,
                                                              **cache))
                    counts["linear"] += 1
    return counts


# ------------------------------------------------------- packed call sites
def project_qkv_decode_packed(hidden_states: torch.Tensor, qkv: W8A8PackedQKV
                              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``_project_qkv_decode_packed`` (llama/paged_attention.py:97-115).

    ``hidden_states`` is ``[1, B, hidden]``; returns q ``[B, H, D]``, k and v
    ``[B, Hkv, D]``.
    """
    return qkv.project(hidden_states)


def project_output_decode_staged(hidden_states: torch.Tensor, o_proj: W8A8Linear
                                 ) -> torch.Tensor:
    """``_project_output_decode_staged`` (llama/paged_attention.py:118-124)."""
    staged = hidden_states[0].contiguous()
    return o_proj(staged).unsqueeze(0)


def packed_mlp_decode(hidden_states: torch.Tensor, mlp: W8A8MLP) -> torch.Tensor:
    """Packed ``LightweightMLP.forward`` branch (lightweight_runner.py:320-383).

    Rows are staged as ``hidden_states[0]`` for a 3-D input (``_decode_rows_layout``,
    :27-35) and the result is ``unsqueeze(0)``-ed, as the reference does.
    """
    rows = hidden_states if hidden_states.dim() == 2 else hidden_states[0]
    if not rows.is_contiguous():
        rows = rows.contiguous()
    return mlp(rows).unsqueeze(0)


def gateup_silu_mul(hidden_states: torch.Tensor, gate_up: W8A8GateUpSiluMul) -> torch.Tensor:
    """Packed gate/up projection followed by ``act_fn(gate) * up``."""
    return gate_up(hidden_states)


def rmsnorm_packed_qkv_decode(hidden_states: torch.Tensor, norm: nn.Module, qkv: W8A8PackedQKV
                              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``_rmsnorm_staged_packed_qkv_decode`` (llama/paged_attention.py:283-305):
    RMSNorm of ``hidden_states[0]``, its per-token quantization and the packed
    QKV product, one kernel at decode shapes (``w8a8_rmsnorm_linear``, the W8A8
    form of ``_rmsnorm_packed_qkv_kernel``, :163-234).  Returns q, k, v views
    like the reference."""
    rows = _rows2(hidden_states)
    if not rows.is_contiguous():
        rows = rows.contiguous()
    return qkv.project_rmsnorm(rows, norm)


def residual_rmsnorm_mlp_decode(hidden_states: torch.Tensor, residual: torch.Tensor,
                                norm: nn.Module, mlp: W8A8MLP
                                ) -> tuple[torch.Tensor, torch.Tensor]:
    """``post_attention_layernorm.residual_norm`` followed by the packed MLP
    (llama/lightweight_runner.py:247-257, 320-383): the residual add, RMSNorm
    and per-token quantization are one kernel; returns ``(residual, mlp_out)``
    with the reference's ``[1, B, H]`` staging for 3-D inputs."""
    three_d = hidden_states.dim() == 3
    rows = _rows2(hidden_states)
    res = _rows2(residual)
    summed, out = mlp.forward_residual_rmsnorm(rows.contiguous(), res.contiguous(), norm)
    if three_d:
        return summed.unsqueeze(0), out.unsqueeze(0)
    return summed, out
