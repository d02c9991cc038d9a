"""W8A8 linear modules for the lightweight LLaMA runner's projection call sites.

Each module owns its quantized weight, packed once into 16x64 MFMA tiles,
and replaces one of the reference's dense call sites:

* :class:`W8A8Linear`            - ``F.linear(x, W, b)`` (O proj,
  ``_project_output_decode_staged``, llama/paged_attention.py:118-124; down
  proj, ``_decode_linear_rows``, llama/lightweight_runner.py:38-54).
* :class:`W8A8PackedQKV`         - the packed QKV projection
  (``PagedLlamaAttention.from_hf`` packing, llama/paged_attention.py:1242-1262;
  ``_project_qkv_decode_packed``, :97-115).
* :class:`W8A8GateUpSiluMul`     - packed gate/up plus ``act_fn(gate) * up``
  (``LightweightMLP`` packed branch, llama/lightweight_runner.py:320-358) in one
  kernel, with the interleaved weight layout of ``_pack_gateup_tensors``
  (:81-92).
* :class:`W8A8RMSNormQuant`      - ``LightweightRMSNorm`` (:225-257) fused with the
  per-token quantization of its output (the int8 rows feed the packed QKV /
  MLP through ``project_i8`` / ``forward_i8``).
* :class:`W8A8MLP`               - gate/up + SiLU*mul + down
  (``LightweightMLP.forward``, :320-383), optionally as an int8 chain where the
  gate/up epilogue requantizes ``h`` with a static (calibrated) scale and the
  down projection consumes int8 directly.

Weights follow ``per_output_weight_qdq`` (nanopointllm/compression/w8a8.py:53-62);
activations are quantized per token (w8a8.py:106-115); results follow the
integer contract of ``integer_linear_per_output_reference`` (w8a8.py:118-139).
Per-row quantization commutes with row packing, so the packed QKV / gate-up
scales are the concatenation / interleave of the per-module scales.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from . import _lib
from . import w8a8 as _w


@dataclass
class PackedW8A8Weight:
    """Per-output int8 weight in packed tiles, with f32 scales and bias."""

    packed: torch.Tensor          # int8, w8a8_packed_bytes(N, K) bytes
    scale: torch.Tensor           # f32 [N] (binary16-representable values)
    bias: torch.Tensor | None     # f32 [N] or None
    out_features: int
    in_features: int
    layout: int = _lib.ROWS_AS_IS

    @classmethod
    def from_int8(cls, qweight: torch.Tensor, scale: torch.Tensor,
                  bias: torch.Tensor | None = None, *,
                  layout: int = _lib.ROWS_AS_IS) -> "PackedW8A8Weight":
        """Pack an already-quantized row-major weight.

        With ``layout == ROWS_INTERLEAVE_HALVES`` the rows of ``qweight`` (and
        ``scale``/``bias``) are ``[gate; up]`` and are packed as g0,u0,g1,u1...
        """
        device = _lib.require_cuda(qweight, scale, bias)
        n, k = qweight.shape
        packed = _w.pack_rows(qweight.contiguous(), layout)
        s = scale.detach().to(device=device, dtype=torch.float32).reshape(-1)
        b = None if bias is None else bias.detach().to(device=device, dtype=torch.float32).reshape(-1)
        if s.numel() != n or (b is not None and b.numel() != n):
            raise ValueError("scale/bias must have one value per output")
        if layout == _lib.ROWS_INTERLEAVE_HALVES:
            s = _interleave_halves(s)
            b = None if b is None else _interleave_halves(b)
        return cls(packed, s.contiguous(), None if b is None else b.contiguous(), n, k, layout)

    @classmethod
    def from_float(cls, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                   layout: int = _lib.ROWS_AS_IS) -> "PackedW8A8Weight":
        """Quantize per output row (``per_output_weight_qdq``) and pack."""
        q, s = _w.quant_rows(weight.detach())
        return cls.from_int8(q, s, bias, layout=layout)


def _packed(build, source: torch.Tensor, weight_cache, cache_key: str, verify_source: bool,
            layout: int = _lib.ROWS_AS_IS):
    if weight_cache is None:
        return build()
    from . import weight_cache as _wc
    return _wc.cached(weight_cache, cache_key, build, source=source,
                      verify_source=verify_source, device=source.device, layout=layout)


def _interleave_halves(v: torch.Tensor) -> torch.Tensor:
    half = v.numel() // 2
    return torch.stack([v[:half], v[half:]], dim=1).reshape(-1)


def _norm_eps(norm: nn.Module) -> float:
    """The epsilon of a LightweightRMSNorm (``variance_epsilon``,
    lightweight_runner.py:229-236) or of a norm that names it ``eps``."""
    for name in ("variance_epsilon", "eps"):
        eps = getattr(norm, name, None)
        if eps is not None:
            return float(eps)
    raise ValueError("the norm module has no epsilon (variance_epsilon or eps)")


def _rows2(hidden_states: torch.Tensor) -> torch.Tensor:
    """``[1, T, hidden]`` (the reference's staged decode layout) or
    ``[T, hidden]`` -> ``[T, hidden]``."""
    if hidden_states.dim() == 3:
        if hidden_states.shape[0] != 1:
            raise ValueError("hidden states must be [1, tokens, hidden] or [tokens, hidden]")
        return hidden_states[0]
    if hidden_states.dim() != 2:
        raise ValueError("hidden states must be [1, tokens, hidden] or [tokens, hidden]")
    return hidden_states


def _linear_parts(module: nn.Module) -> tuple[torch.Tensor, torch.Tensor | None]:
    return module.weight, getattr(module, "bias", None)


class W8A8Linear(nn.Module):
    """``F.linear(x, W, b)`` with A8 activations and per-output W8.

    By default activations are quantized per token (dynamic).  A SmoothQuant
    ``smooth`` vector [K] (the input smoothing scales of
    ``apply_smoothquant_transform``, w8a8.py:373-414, applied to the weight
    before it was quantized) makes the forward divide x by it first, and a
    ``static_scale`` replaces the per-token scale (static A8, w8a8.py:94-103):
    both run fused in the activation prologue kernel before the int8-in
    product.
    """

    def __init__(self, weight: PackedW8A8Weight, *, smooth: torch.Tensor | None = None,
                 static_scale: float | None = None) -> None:
        super().__init__()
        self.weight_q = weight
        self.in_features = weight.in_features
        self.out_features = weight.out_features
        if smooth is not None and smooth.numel() != weight.in_features:
            raise ValueError("smoothing scales must have one value per input channel")
        if static_scale is not None and not static_scale > 0:
            raise ValueError("quantization scale must be positive")
        self.register_buffer("smooth", None if smooth is None else smooth.detach().reshape(-1))
        self.static_scale = None if static_scale is None else float(static_scale)

    @classmethod
    def from_linear(cls, linear: nn.Module, *, smooth: torch.Tensor | None = None,
                    static_scale: float | None = None, weight_cache=None, cache_key: str = "",
                    verify_source: bool = False) -> "W8A8Linear":
        """Quantize and pack ``linear``'s weight, or load it from the packed
        weight cache directory ``weight_cache`` under ``cache_key``."""
        w, b = _linear_parts(linear)
        packed = _packed(lambda: PackedW8A8Weight.from_float(w, b), w, weight_cache, cache_key,
                         verify_source)
        return cls(packed, smooth=smooth, static_scale=static_scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        p = self.weight_q
        if self.smooth is None and self.static_scale is None:
            return _w.linear_dynamic(x, p.packed, p.scale, p.bias, p.out_features,
                                     in_features=p.in_features)
        if x.shape[-1] != p.in_features:
            raise ValueError("linear input/weight shapes do not match")
        out = _w.prologue_quant(x, smooth=self.smooth, static_scale=self.static_scale)
        return _w.linear_i8in(out.q, out.scale.reshape(-1), p.packed, p.scale, p.bias,
                              p.out_features, out_dtype=x.dtype, in_features=p.in_features)

    def forward_i8(self, xq: torch.Tensor, x_scale: torch.Tensor,
                   out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """Same product for int8 activations with per-row scales."""
        p = self.weight_q
        return _w.linear_i8in(xq, x_scale, p.packed, p.scale, p.bias, p.out_features,
                              out_dtype=out_dtype, in_features=p.in_features)

    def forward_residual(self, x: torch.Tensor, residual: torch.Tensor) -> _w.ResidualOutput:
        """``residual + self(x)`` in the activation dtype with the RMSNorm
        chunk sums of the result (``linear_residual``): the residual add of a
        decoder layer after o_proj / down_proj (lightweight_runner.py:247-257,
        552) in this linear's epilogue.  Dynamic per-token activations only."""
        if self.smooth is not None or self.static_scale is not None:
            raise ValueError("the residual-add epilogue takes per-token dynamic activations")
        p = self.weight_q
        return _w.linear_residual(x, p.packed, p.scale, p.bias, p.out_features, residual,
                                  in_features=p.in_features)

    def forward_i8_residual(self, xq: torch.Tensor, x_scale: torch.Tensor,
                            residual: torch.Tensor) -> _w.ResidualOutput:
        """:meth:`forward_residual` on int8 activations with per-row scales."""
        p = self.weight_q
        return _w.linear_i8in_residual(xq, x_scale, p.packed, p.scale, p.bias, p.out_features,
                                       residual, in_features=p.in_features)

    def accumulators(self, x: torch.Tensor) -> torch.Tensor:
        """Raw int32 accumulators of ``forward`` (for exactness checks)."""
        p = self.weight_q
        return _w.linear_dynamic(x, p.packed, p.scale, None, p.out_features,
                                 epilogue=_lib.EPI_I32, in_features=p.in_features)


class W8A8PackedQKV(nn.Module):
    """Packed ``[Wq; Wk; Wv]`` projection (paged_attention.py:1242-1262)."""

    def __init__(self, q_proj: nn.Module, k_proj: nn.Module, v_proj: nn.Module, *,
                 num_heads: int, num_kv_heads: int, head_dim: int, weight_cache=None,
                 cache_key: str = "packed_qkv", verify_source: bool = False) -> None:
        super().__init__()
        parts = [_linear_parts(m) for m in (q_proj, k_proj, v_proj)]
        weight = torch.cat([w for w, _ in parts], dim=0)
        if all(b is None for _, b in parts):
            bias = None
        else:
            bias = torch.cat([b if b is not None else w.new_zeros(w.shape[0])
                              for w, b in parts], dim=0)
        self.linear = W8A8Linear(_packed(lambda: PackedW8A8Weight.from_float(weight, bias),
                                         weight, weight_cache, cache_key, verify_source))
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self.linear(hidden_states)

    def project(self, hidden_states: torch.Tensor
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``_project_qkv_decode_packed`` (paged_attention.py:97-115) semantics."""
        return self._split(self.linear(_rows2(hidden_states)))

    def project_i8(self, xq: torch.Tensor, x_scale: torch.Tensor, *,
                   out_dtype: torch.dtype = torch.float16
                   ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """As :meth:`project` for int8 rows with per-row scales (the output of
        the fused RMSNorm + quantization prologue)."""
        return self._split(self.linear.forward_i8(xq, x_scale, out_dtype=out_dtype))

    def project_rmsnorm(self, hidden_states: torch.Tensor, norm: nn.Module
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``_rmsnorm_staged_packed_qkv_decode`` (paged_attention.py:283-305):
        ``norm`` (a LightweightRMSNorm / LlamaRMSNorm) applied to the rows,
        then the packed QKV projection, one kernel at decode shapes."""
        staged = _rows2(hidden_states)
        lin = self.linear.weight_q
        out = _w.rmsnorm_linear(staged, norm.weight, _norm_eps(norm), lin.packed, lin.scale,
                                lin.bias, lin.out_features, in_features=lin.in_features)
        return self._split(out.y)

    def project_rmsnorm_residual(self, hidden_states: torch.Tensor, residual: torch.Tensor,
                                 norm: nn.Module
                                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """As :meth:`project_rmsnorm` on ``dtype(hidden_states + residual)``
        (``residual_norm``, lightweight_runner.py:247-257): the add runs in the
        same launch.  Returns ``(q, k, v, hidden_states + residual)``."""
        lin = self.linear.weight_q
        out = _w.rmsnorm_linear(_rows2(hidden_states), norm.weight, _norm_eps(norm), lin.packed,
                                lin.scale, lin.bias, lin.out_features,
                                residual=_rows2(residual), in_features=lin.in_features)
        q, k, v = self._split(out.y)
        return q, k, v, out.residual

    def project_rmsnorm_ss(self, hidden_states: torch.Tensor, ss_parts: torch.Tensor,
                           norm: nn.Module
                           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """:meth:`project_rmsnorm` on rows that a residual-add linear wrote
        with their RMSNorm chunk sums ``ss_parts``: the one-kernel decode
        route reads the sums instead of summing the rows (the same bits)."""
        lin = self.linear.weight_q
        out = _w.rmsnorm_linear(_rows2(hidden_states), norm.weight, _norm_eps(norm), lin.packed,
                                lin.scale, lin.bias, lin.out_features,
                                in_features=lin.in_features, ss_parts=ss_parts)
        return self._split(out.y)

    def _split(self, qkv: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        q_size = self.num_heads * self.head_dim
        kv_size = self.num_kv_heads * self.head_dim
        q, k, v = torch.split(qkv, (q_size, kv_size, kv_size), dim=-1)
        return (q.view(-1, self.num_heads, self.head_dim),
                k.view(-1, self.num_kv_heads, self.head_dim),
                v.view(-1, self.num_kv_heads, self.head_dim))


class W8A8GateUpSiluMul(nn.Module):
    """Packed gate/up projection fused with ``act_fn(gate) * up``.

    Weights are packed in the reference's interleave layout (g0,u0,g1,u1...),
    so each 16-output tile carries 8 (gate, up) pairs and the epilogue emits
    ``SiLU(g) * u`` with the reference's binary16 roundings
    (lightweight_runner.py:344-358).
    """

    def __init__(self, gate_proj: nn.Module, up_proj: nn.Module, *, weight_cache=None,
                 cache_key: str = "packed_gate_up", verify_source: bool = False) -> None:
        super().__init__()
        (wg, bg), (wu, bu) = _linear_parts(gate_proj), _linear_parts(up_proj)
        weight = torch.cat([wg, wu], dim=0)
        if bg is None and bu is None:
            bias = None
        else:
            bias = torch.cat([bg if bg is not None else wg.new_zeros(wg.shape[0]),
                              bu if bu is not None else wu.new_zeros(wu.shape[0])])
        self.weight_q = _packed(
            lambda: PackedW8A8Weight.from_float(weight, bias, layout=_lib.ROWS_INTERLEAVE_HALVES),
            weight, weight_cache, cache_key, verify_source, _lib.ROWS_INTERLEAVE_HALVES)
        self.intermediate = wg.shape[0]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        p = self.weight_q
        return _w.linear_dynamic(x, p.packed, p.scale, p.bias, p.out_features,
                                 epilogue=_lib.EPI_SILU_MUL, in_features=p.in_features)

    def forward_q8(self, x: torch.Tensor, h_scale: float) -> torch.Tensor:
        """``quantize_symmetric(SiLU(g) * u, h_scale)`` as int8 (static requant)."""
        p = self.weight_q
        return _w.linear_dynamic(x, p.packed, p.scale, p.bias, p.out_features,
                                 epilogue=_lib.EPI_SILU_MUL_Q8, y_scale=h_scale,
                                 in_features=p.in_features)

    def forward_i8(self, xq: torch.Tensor, x_scale: torch.Tensor, *,
                   out_dtype: torch.dtype = torch.float16,
                   h_scale: float | None = None) -> torch.Tensor:
        """``SiLU(g) * u`` from int8 rows with per-row scales; with ``h_scale``
        the result is requantized to int8 as in :meth:`forward_q8`."""
        p = self.weight_q
        if h_scale is None:
            return _w.linear_i8in(xq, x_scale, p.packed, p.scale, p.bias, p.out_features,
                                  epilogue=_lib.EPI_SILU_MUL, out_dtype=out_dtype,
                                  inter_dtype=out_dtype, in_features=p.in_features)
        return _w.linear_i8in(xq, x_scale, p.packed, p.scale, p.bias, p.out_features,
                              epilogue=_lib.EPI_SILU_MUL_Q8, out_dtype=torch.int8,
                              y_scale=h_scale, inter_dtype=out_dtype,
                              in_features=p.in_features)

    def forward_two_phase(self, x: torch.Tensor, x_scale: torch.Tensor | None = None, *,
                          out_dtype: torch.dtype | None = None) -> "_w.TwoPhaseOutput":
        """``SiLU(g) * u`` and its per-token dynamic int8 quantization in two
        phases (the epilogue keeps each row's |h|max per weight block, a
        second kernel quantizes): ``(h, hq, scale)``, ``hq``/``scale`` exactly
        ``dynamic_per_token_activation_qdq``'s integer part of ``h``.  ``x``
        is 16-bit (quantized per token) or int8 with ``x_scale``."""
        p = self.weight_q
        if out_dtype is None and x.dtype == torch.int8:
            out_dtype = torch.float16
        return _w.gateup_silu_mul_two_phase(x, p.packed, p.scale, p.bias, p.out_features,
                                            x_scale=x_scale, h_dtype=out_dtype,
                                            in_features=p.in_features)

    def accumulators(self, x: torch.Tensor) -> torch.Tensor:
        """int32 accumulators in packed (interleaved) column order."""
        p = self.weight_q
        return _w.linear_dynamic(x, p.packed, p.scale, None, p.out_features,
                                 epilogue=_lib.EPI_I32, in_features=p.in_features)


class W8A8MLP(nn.Module):
    """LLaMA MLP ``down(SiLU(gate(x)) * up(x))`` on the W8A8 kernels.

    With ``h_scale`` (a calibrated static scale for ``h``, e.g. from
    ``static_activation_scale``) the gate/up kernel writes int8 ``h`` and the
    down projection consumes it directly (int8-in chain).  Otherwise ``h`` is
    quantized per token (dynamic): by default the down projection quantizes
    the 16-bit ``h`` itself (inside its one launch at M <= 4); with
    ``two_phase`` the gate/up epilogue keeps each row's |h|max per weight
    block and a second kernel writes int8 ``h`` for the int8-in down
    projection.  Both dynamic forms give the same bits; measured on MI355X at
    LLaMA-7B shapes the two-phase chain ties at M = 8 and is 2-3 us slower
    per layer at M <= 4, where it adds a launch.
    """

    def __init__(self, gate_proj: nn.Module, up_proj: nn.Module, down_proj: nn.Module, *,
                 h_scale: float | None = None, weight_cache=None, cache_prefix: str = "",
                 verify_source: bool = False, two_phase: bool = False) -> None:
        super().__init__()
        self.gate_up = W8A8GateUpSiluMul(gate_proj, up_proj, weight_cache=weight_cache,
                                         cache_key=cache_prefix + "packed_gate_up",
                                         verify_source=verify_source)
        self.down = W8A8Linear.from_linear(down_proj, weight_cache=weight_cache,
                                           cache_key=cache_prefix + "down_proj",
                                           verify_source=verify_source)
        self.h_scale = h_scale
        self.two_phase = two_phase
        self._h_rows_buf: dict[tuple[torch.device, float], torch.Tensor] = {}
        self._h_rows_keep: list[torch.Tensor] = []

    def _h_rows(self, hq: torch.Tensor) -> torch.Tensor:
        """The static h scale once per row of ``hq``: a prefix of one filled
        buffer per device and scale (a fill per call would add kernels to
        every decode step; a captured step finds the buffer made by its
        warm-up calls).  The buffer grows geometrically and the outgrown ones
        are kept, since a captured graph may still read them."""
        m = hq.numel() // hq.shape[-1] if hq.numel() else 0
        key = (hq.device, float(self.h_scale))
        buf = self._h_rows_buf.get(key)
        if buf is None or buf.numel() < m:
            size = max(m, 16, 2 * (0 if buf is None else buf.numel()))
            buf = torch.full((size,), self.h_scale, dtype=torch.float32, device=hq.device)
            self._h_rows_keep.append(buf)
            self._h_rows_buf[key] = buf
        return buf[:m]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.h_scale is None:
            if self.two_phase:
                out = self.gate_up.forward_two_phase(x)
                return self.down.forward_i8(out.hq, out.scale.reshape(-1), out_dtype=x.dtype)
            return self.down(self.gate_up(x))
        hq = self.gate_up.forward_q8(x, self.h_scale)
        return self.down.forward_i8(hq, self._h_rows(hq), out_dtype=x.dtype)

    def forward_residual_rmsnorm(self, hidden_states: torch.Tensor, residual: torch.Tensor,
                                 norm: nn.Module) -> tuple[torch.Tensor, torch.Tensor]:
        """``post_attention_layernorm.residual_norm`` then the MLP
        (lightweight_runner.py:247-257, 320-383), with the residual add and
        RMSNorm inside the gate/up launch at decode shapes.  Returns
        ``(hidden_states + residual, mlp output)``.

        ``two_phase`` has no effect here: this route always hands the 16-bit
        ``h`` to the down projection, which quantizes it per token in its own
        launch.  The two-phase route gives the same bits (it quantizes the
        same ``h`` with the same per-token scales) and would add a launch to
        this one, since the fused norm kernel does not write the partial
        row maxima."""
        p = self.gate_up.weight_q
        epi = _lib.EPI_SILU_MUL if self.h_scale is None else _lib.EPI_SILU_MUL_Q8
        first = _w.rmsnorm_linear(hidden_states, norm.weight, _norm_eps(norm), p.packed, p.scale,
                                  p.bias, p.out_features, residual=residual, epilogue=epi,
                                  y_scale=0.0 if self.h_scale is None else self.h_scale,
                                  in_features=p.in_features)
        if self.h_scale is None:
            return first.residual, self.down(first.y)
        return first.residual, self.down.forward_i8(first.y, self._h_rows(first.y),
                                                    out_dtype=hidden_states.dtype)

    def forward_rmsnorm_ss_residual(self, hidden_states: torch.Tensor, ss_parts: torch.Tensor,
                                    norm: nn.Module) -> _w.ResidualOutput:
        """``hidden_states + mlp(norm(hidden_states))`` for rows that a
        residual-add linear wrote with their RMSNorm chunk sums ``ss_parts``
        (the o_proj of :meth:`W8A8Linear.forward_residual`): the norm and
        gate/up run as one launch that reads the sums, and down adds the
        rows back in its epilogue and returns the next norm's sums
        (lightweight_runner.py:247-257, 320-383, 552)."""
        p = self.gate_up.weight_q
        epi = _lib.EPI_SILU_MUL if self.h_scale is None else _lib.EPI_SILU_MUL_Q8
        h = _w.rmsnorm_linear(hidden_states, norm.weight, _norm_eps(norm), p.packed, p.scale,
                              p.bias, p.out_features, epilogue=epi,
                              y_scale=0.0 if self.h_scale is None else self.h_scale,
                              in_features=p.in_features, ss_parts=ss_parts).y
        if self.h_scale is None:
            return self.down.forward_residual(h, hidden_states)
        return self.down.forward_i8_residual(h, self._h_rows(h), hidden_states)

    def forward_i8(self, xq: torch.Tensor, x_scale: torch.Tensor, *,
                   out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """The MLP on int8 rows with per-row scales (the output of the fused
        residual-add + RMSNorm + quantization prologue)."""
        if self.h_scale is None:
            if self.two_phase:
                out = self.gate_up.forward_two_phase(xq, x_scale, out_dtype=out_dtype)
                return self.down.forward_i8(out.hq, out.scale.reshape(-1), out_dtype=out_dtype)
            return self.down(self.gate_up.forward_i8(xq, x_scale, out_dtype=out_dtype))
        hq = self.gate_up.forward_i8(xq, x_scale, out_dtype=out_dtype, h_scale=self.h_scale)
        return self.down.forward_i8(hq, self._h_rows(hq), out_dtype=out_dtype)


class W8A8RMSNormQuant(nn.Module):
    """``LightweightRMSNorm`` (lightweight_runner.py:225-257) fused with the
    per-token int8 quantization of its output, for norms whose only consumer
    is a W8A8 projection (input_layernorm -> packed QKV,
    post_attention_layernorm -> packed gate/up).

    ``forward(h) -> (xq, s_x)``; ``residual_norm(h, r) -> (h + r, xq, s_x)``.
    The weight keeps the norm's dtype: a binary32 weight promotes the
    normalized rows to binary32 before quantization, as torch does.
    """

    def __init__(self, norm: nn.Module) -> None:
        super().__init__()
        self.weight = norm.weight
        self.variance_epsilon = _norm_eps(norm)

    def forward(self, hidden_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return _w.rmsnorm_quant(hidden_states, self.weight, self.variance_epsilon)

    def residual_norm(self, hidden_states: torch.Tensor, residual: torch.Tensor
                      ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return _w.rmsnorm_quant(hidden_states, self.weight, self.variance_epsilon,
                                residual=residual)
