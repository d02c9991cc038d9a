"""A LLaMA decoder stack on the W8A8 kernels, in the shape of the reference's
``LightweightLlamaLayer`` / ``LightweightLlamaRunner``
(nanopointllm/llama/lightweight_runner.py:421-737).

Per layer, every projection runs on int8 and every norm feeding one is fused
with the quantization of its output:

1-2. ``input_layernorm``, per-token int8 quantization and the packed
   ``[Wq; Wk; Wv]`` projection (``w8a8_rmsnorm_linear``): one kernel at decode
   shapes, the W8A8 form of ``_rmsnorm_packed_qkv_kernel`` /
   ``_rmsnorm_staged_packed_qkv_decode`` (llama/paged_attention.py:163-234,
   283-305); for prefill the norm kernel writes the int8 rows in the GEMM's
   tiles.  The packed product serves prefill too (the reference's prefill
   runs three projections, paged_attention.py:1349-1352; one packed product
   is the same numbers, since quantization is per token and per output row).
   Every route sums the norm's squares in the same order, so a row's result
   does not depend on the batch it runs in;
3. the attention core, supplied by the caller (rotary, KV cache and the
   attention kernel are not part of the W8A8 path):
   ``core(q [T, H, D], k [T, Hkv, D], v [T, Hkv, D], layer_index, state)``
   returns the context ``[T, H * D]``;
4. ``o_proj`` as a W8A8 linear (paged_attention.py:1376, 1488);
5-6. residual add + ``post_attention_layernorm`` (``residual_norm``,
   lightweight_runner.py:247-257) + int8 quantization + packed gate/up with
   the SiLU*mul epilogue, one kernel at decode shapes, then down (binary16
   ``h``, or the int8 chain with a calibrated ``h`` scale)
   (lightweight_runner.py:320-383);
7. the final residual add in the activation dtype, as the reference does.

At decode batches (at most 8 rows) the residual adds move into the
epilogues of o_proj and down, which also write the RMSNorm sums of squares
of their rows per 8 columns; the next norm + projection launch reads those
sums instead of summing the rows in every workgroup
(:meth:`W8A8LlamaLayer.forward_stream`), with the same bits.

After the last layer, its residual add and the final ``norm``
(``LightweightRMSNorm``, lightweight_runner.py:609, 675) run as one launch of
the activation prologue, the same kernel and formula as the in-layer norms,
in front of the LM head, whose decode batches (at most 16 rows) run as the
dense 16-bit GEMV of :mod:`nanopointllm_amd.lm_head` on the module's own
weight.

The stack is inference-only (no autograd).  Nothing on it synchronizes with
the host or allocates outside torch's allocator, so a decode step can be
captured into a HIP graph;
:class:`DecodeGraphBucket` follows the reference's strict capture/replay
wrapper (nanopointllm/engine/cuda_graph.py:17-52).
"""
from __future__ import annotations

from typing import Any, Callable

import torch
import torch.nn as nn

from . import w8a8 as _w
from .inject import inject_w8a8
from .lm_head import DecodeLMHead
from .linear import W8A8Linear, W8A8MLP, W8A8PackedQKV, _norm_eps

AttentionCore = Callable[[torch.Tensor, torch.Tensor, torch.Tensor, int, Any], torch.Tensor]


def _rows(hidden_states: torch.Tensor) -> torch.Tensor:
    """``[1, T, hidden]`` (the reference's flattened-token layout) or
    ``[T, hidden]`` -> contiguous ``[T, hidden]``."""
    if hidden_states.dim() == 3:
        if hidden_states.shape[0] != 1:
            raise ValueError("hidden states must be [1, tokens, hidden] or [tokens, hidden]")
        hidden_states = hidden_states[0]
    if hidden_states.dim() != 2:
        raise ValueError("hidden states must be [1, tokens, hidden] or [tokens, hidden]")
    return hidden_states if hidden_states.is_contiguous() else hidden_states.contiguous()


class W8A8LlamaLayer(nn.Module):
    """One decoder layer (lightweight_runner.py:421-560) on W8A8 projections.

    ``hf_layer`` must already carry the W8A8 modules of :func:`inject_w8a8`
    (``self_attn.w8a8_qkv``, a W8A8 ``self_attn.o_proj``, ``mlp.w8a8_mlp``).
    """

    def __init__(self, hf_layer: nn.Module, layer_index: int, attention_core: AttentionCore
                 ) -> None:
        super().__init__()
        attn, mlp = hf_layer.self_attn, hf_layer.mlp
        qkv = getattr(attn, "w8a8_qkv", None)
        w8a8_mlp = getattr(mlp, "w8a8_mlp", None)
        if not isinstance(qkv, W8A8PackedQKV) or not isinstance(attn.o_proj, W8A8Linear) \
                or not isinstance(w8a8_mlp, W8A8MLP):
            raise ValueError(f"layer {layer_index} has no W8A8 modules; run inject_w8a8 first")
        self.layer_index = layer_index
        self.input_layernorm = hf_layer.input_layernorm
        self.post_attention_layernorm = hf_layer.post_attention_layernorm
        self.qkv = qkv
        self.o_proj = attn.o_proj
        self.mlp = w8a8_mlp
        self.attention_core = attention_core

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor, attention_state: Any = None) -> torch.Tensor:
        rows = _rows(hidden_states)
        # RMSNorm -> packed QKV and residual add + RMSNorm -> gate/up each run
        # as one launch at decode shapes (w8a8_rmsnorm_linear).
        q, k, v = self.qkv.project_rmsnorm(rows, self.input_layernorm)
        context = self.attention_core(q, k, v, self.layer_index, attention_state)
        attn_out = self.o_proj(context)
        residual, mlp_out = self.mlp.forward_residual_rmsnorm(attn_out, rows,
                                                              self.post_attention_layernorm)
        out = residual + mlp_out
        return out.unsqueeze(0) if hidden_states.dim() == 3 else out

    @torch.no_grad()
    def forward_carry(self, hidden_states: torch.Tensor, residual: torch.Tensor | None,
                      attention_state: Any = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer with its final residual add left to the caller: returns
        ``(mlp_out, residual)``, whose binary16 / bfloat16 sum is what
        :meth:`forward` returns.  With ``residual`` given, the layer's input
        is ``dtype(hidden_states + residual)``, formed in the RMSNorm + packed
        QKV launch; a rounded add of two 16-bit values is the same single
        rounding wherever it runs, so a stack of ``forward_carry`` calls gives
        the bits of a stack of ``forward`` calls with one launch fewer per
        layer."""
        rows = _rows(hidden_states)
        if residual is None:
            q, k, v = self.qkv.project_rmsnorm(rows, self.input_layernorm)
            layer_in = rows
        else:
            q, k, v, layer_in = self.qkv.project_rmsnorm_residual(rows, _rows(residual),
                                                                  self.input_layernorm)
        context = self.attention_core(q, k, v, self.layer_index, attention_state)
        attn_out = self.o_proj(context)
        residual, mlp_out = self.mlp.forward_residual_rmsnorm(attn_out, layer_in,
                                                              self.post_attention_layernorm)
        return mlp_out, residual


    @torch.no_grad()
    def forward_stream(self, hidden_states: torch.Tensor, ss_parts: torch.Tensor | None,
                       attention_state: Any = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The layer on the residual stream itself: ``hidden_states`` are the
        layer's input rows with every residual add done, ``ss_parts`` their
        RMSNorm sums of squares per 8 columns when a residual-add linear wrote
        them (None for rows from elsewhere).  o_proj and down add the
        residual in their epilogues (lightweight_runner.py:247-257, 552) and
        return the sums their rows' norms need, so the RMSNorm launches in
        front of the packed QKV and gate/up read those sums instead of summing
        every row in every workgroup.  Returns ``(output rows, their sums)``;
        the bits are those of :meth:`forward`.  Needs per-token dynamic
        activations on o_proj."""
        rows = _rows(hidden_states)
        if ss_parts is None:
            q, k, v = self.qkv.project_rmsnorm(rows, self.input_layernorm)
        else:
            q, k, v = self.qkv.project_rmsnorm_ss(rows, ss_parts, self.input_layernorm)
        context = self.attention_core(q, k, v, self.layer_index, attention_state)
        summed, parts = self.o_proj.forward_residual(context, rows)
        out = self.mlp.forward_rmsnorm_ss_residual(summed, parts, self.post_attention_layernorm)
        return out.y, out.ss_parts


class W8A8LlamaRunner(nn.Module):
    """``LightweightLlamaRunner`` (lightweight_runner.py:563-737) with W8A8
    decoder layers: ``embed_tokens`` -> layers -> ``norm`` -> ``lm_head``.

    The final norm (residual add included) runs on the activation prologue
    kernel when its weight has the activations' dtype, else as the model's
    own module; the LM head stays a linear in the model's dtype (it is not a
    W8A8 linear in the reference either).  ``inject`` installs the W8A8
    modules first (``h_scales`` and ``weight_cache`` as in :func:`inject_w8a8`).
    """

    def __init__(self, hf_model: nn.Module, attention_core: AttentionCore, *,
                 inject: bool = True, h_scales: dict[int, float] | None = None,
                 weight_cache=None) -> None:
        super().__init__()
        if inject:
            inject_w8a8(hf_model, h_scales=h_scales, weight_cache=weight_cache)
        model = hf_model.model if hasattr(hf_model, "model") else hf_model
        self.hf_model = hf_model
        self.embed_tokens = model.embed_tokens
        self.layers = nn.ModuleList([W8A8LlamaLayer(layer, i, attention_core)
                                     for i, layer in enumerate(model.layers)])
        self.norm = model.norm
        # Decode batches take the dense GEMV (lm_head.DecodeLMHead); the
        # reference calls the module's F.linear (lightweight_runner.py:676-681).
        self.lm_head = DecodeLMHead(hf_model.lm_head)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor | None = None, *,
                inputs_embeds: torch.Tensor | None = None,
                attention_state: Any = None) -> torch.Tensor:
        if inputs_embeds is None:
            if input_ids is None:
                raise ValueError("input_ids or inputs_embeds is required")
            hidden_states = self.embed_tokens(input_ids)
        else:
            hidden_states = inputs_embeds
        shape = hidden_states.shape
        rows = _rows(hidden_states)
        if self.stream_route(rows):
            # Decode: o_proj and down add the residual in their epilogues and
            # hand the next norm its sums of squares (forward_stream).
            hidden, parts = rows, None
            for layer in self.layers:
                hidden, parts = layer.forward_stream(hidden, parts, attention_state)
            return self.lm_head(self.final_norm(hidden, None).view(shape))
        # Each layer's final residual add (lightweight_runner.py:552) runs in
        # the next layer's RMSNorm + QKV launch; the last one in the final norm's.
        hidden, residual = rows, None
        for layer in self.layers:
            hidden, residual = layer.forward_carry(hidden, residual, attention_state)
        return self.lm_head(self.final_norm(hidden, residual).view(shape))

    def stream_route(self, rows: torch.Tensor) -> bool:
        """Whether a forward over ``rows`` takes :meth:`W8A8LlamaLayer.forward_stream`:
        decode batches (at most 8 rows, where the RMSNorm + projection runs as
        one kernel per CU and the sums spare each CU the row sums) of 16-bit
        rows, with per-token dynamic o_proj activations.  Both routes give the
        same bits; larger batches keep the residual adds in the norm
        launches, which sum the rows once per row, not once per CU."""
        return (rows.shape[0] <= 8 and rows.dtype in (torch.float16, torch.bfloat16)
                and all(layer.o_proj.smooth is None and layer.o_proj.static_scale is None
                        for layer in self.layers))

    def final_norm(self, hidden: torch.Tensor, residual: torch.Tensor | None) -> torch.Tensor:
        """``norm(dtype(hidden + residual))`` for ``[T, hidden]`` rows
        (lightweight_runner.py:247-257, 675): one launch of the activation
        prologue, whose normalized rows are the output (its int8 rows are not
        used).  Rows that are not binary16 / bfloat16, or a norm weight of
        another dtype than the rows', run the model's own module."""
        w = self.norm.weight
        if hidden.dtype not in (torch.float16, torch.bfloat16) or w.dtype != hidden.dtype:
            return self.norm(hidden if residual is None else residual + hidden)
        return _w.prologue_quant(hidden, norm_weight=w, eps=_norm_eps(self.norm),
                                 residual=residual, return_rows=True).rows


class DecodeGraphBucket:
    """Strict capture / replay of one fixed-shape decode step
    (nanopointllm/engine/cuda_graph.py:17-52): ``capture(forward)`` warms the
    kernels up twice, captures one call and returns its static output;
    ``replay()`` reruns the captured kernels on whatever the static inputs
    hold.  Errors propagate; there is no eager fallback."""

    def __init__(self, device: torch.device | str = "cuda") -> None:
        self.device = torch.device(device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.static_output: torch.Tensor | None = None

    @property
    def captured(self) -> bool:
        return self.graph is not None

    def capture(self, forward: Callable[[], torch.Tensor]) -> torch.Tensor:
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("decode graph capture needs a GPU")
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                forward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = forward()
        self.graph, self.static_output = graph, out
        return out

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("decode graph bucket has not been captured")
        self.graph.replay()
        return self.static_output
