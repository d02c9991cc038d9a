"""W8A8 numerical contract on the GPU (HIP kernels through libw8a8_gfx950.so).

Mirrors the function API of ``nanopointllm.compression.w8a8``
(nanopointllm/compression/w8a8.py) for CUDA tensors: same names, same
argument meaning, same results, same error messages.  Every integer result is
produced by the HIP kernels; torch is used only for device memory, reshapes
and the trivial elementwise QDQ reconstruction (``q * s``).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
from functools import lru_cache
from typing import Any, NamedTuple

import torch

from . import _lib

_F16_TINY = torch.finfo(torch.float16).tiny  # 2**-14


@dataclass(frozen=True)
class W8A8Contract:
    """Same fields and values as the reference contract (w8a8.py:14-30)."""

    weight_bits: int = 8
    activation_bits: int = 8
    symmetric_min: int = -127
    symmetric_max: int = 127
    rounding: str = "round_to_nearest_ties_to_even"
    scale_storage: str = "float16"
    accumulator: str = "signed_int32"
    bias: str = "floating_point_after_dequantization"
    nonlinear_norm_residual: str = "bf16_or_fp16"

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)


CONTRACT = W8A8Contract()


# ---------------------------------------------------------------- low level
@lru_cache(maxsize=1024)
def packed_bytes(rows: int, k: int) -> int:
    return int(_lib.load().w8a8_packed_bytes(rows, k))


@lru_cache(maxsize=1024)
def workspace_bytes(m: int, k: int) -> int:
    return int(_lib.load().w8a8_workspace_bytes(m, k))


def _rows_view(x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """2-D [rows, K] view with unit column stride, plus its leading dimension."""
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if x2.shape[0] > 0 and (x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < k)):
        x2 = x2.contiguous()
    ld = x2.stride(0) if x2.shape[0] > 1 else max(k, 1)
    return x2, ld


def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-row int8 quantization of ``x[..., K]``.

    Returns ``(q int8 [..., K], scales f32 [...])``; the scale of each row is
    ``scale_from_absmax(|row|.amax())`` (w8a8.py:46-50, 106-115).
    """
    device = _lib.require_cuda(x)
    x2, ldx = _rows_view(x)
    rows, k = x2.shape
    q = torch.empty((rows, k), dtype=torch.int8, device=device)
    s = torch.empty((rows,), dtype=torch.float32, device=device)
    if rows:
        lib = _lib.load()
        _lib.check(lib.w8a8_quant_rows(x2.data_ptr(), _lib.dtype_code(x2.dtype), rows, k, ldx,
                                       q.data_ptr(), max(k, 1), s.data_ptr(),
                                       _lib.stream_handle(device)), "w8a8_quant_rows")
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def quant_rows_scaled(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``quantize_symmetric`` with one scale per tensor or per row (no checks)."""
    device = _lib.require_cuda(x, scale)
    x2, ldx = _rows_view(x)
    rows, k = x2.shape
    s = scale.detach().to(device=device, dtype=torch.float32).contiguous()
    if s.numel() == 1:
        stride = 0
    elif s.numel() == rows:
        stride = 1
    else:
        raise ValueError("scale must be per-tensor or one value per row of the last dimension")
    q = torch.empty((rows, k), dtype=torch.int8, device=device)
    if rows:
        lib = _lib.load()
        _lib.check(lib.w8a8_quant_rows_scaled(x2.data_ptr(), _lib.dtype_code(x2.dtype), rows, k,
                                              ldx, s.data_ptr(), stride, q.data_ptr(),
                                              max(k, 1), _lib.stream_handle(device)),
                   "w8a8_quant_rows_scaled")
    return q.reshape(x.shape)


def pack_rows(q: torch.Tensor, layout: int = _lib.ROWS_AS_IS) -> torch.Tensor:
    """Pack int8 ``q[rows, K]`` into 16x64 MFMA tiles (flat int8 tensor)."""
    device = _lib.require_cuda(q)
    if q.dtype != torch.int8 or q.dim() != 2:
        raise ValueError("pack_rows expects a 2-D int8 tensor")
    if q.stride(-1) != 1:
        q = q.contiguous()
    rows, k = q.shape
    out = torch.empty((packed_bytes(rows, k),), dtype=torch.int8, device=device)
    if rows and k:
        lib = _lib.load()
        _lib.check(lib.w8a8_pack_rows(q.data_ptr(), rows, k, q.stride(0) if rows > 1 else k,
                                      layout, out.data_ptr(), _lib.stream_handle(device)),
                   "w8a8_pack_rows")
    return out


def _workspace(m: int, k: int, device: torch.device) -> torch.Tensor:
    return torch.empty((max(workspace_bytes(m, k), 16),), dtype=torch.uint8, device=device)


def _check_operands(k: int, w_packed: torch.Tensor, w_scale: torch.Tensor | None,
                    bias: torch.Tensor | None, n: int, in_features: int | None) -> None:
    """Host checks before any launch: the C ABI only sees pointers, so an
    activation whose K differs from the packed weight's, or a weight, scale or
    bias buffer shorter than ``n`` x ``k`` implies, must be refused here (the
    reference's F.linear raises on the same mismatch, w8a8.py:126-127)."""
    if in_features is not None and k != in_features:
        raise ValueError("linear input/weight shapes do not match")
    if w_packed.dtype != torch.int8 or not w_packed.is_contiguous():
        raise ValueError("packed weight must be a contiguous int8 tensor")
    if n < 0 or w_packed.numel() < packed_bytes(n, k):
        raise ValueError("linear input/weight shapes do not match")
    for name, t in (("weight scale", w_scale), ("bias", bias)):
        if t is None:
            continue
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor")
        if t.numel() < n:
            raise ValueError(f"{name} must have one value per output")


def gemm_i32(xq: torch.Tensor, w_packed: torch.Tensor, n: int, *,
             in_features: int | None = None) -> torch.Tensor:
    """Exact ``int32(xq) @ int32(wq).T`` for packed ``wq`` ([..., K] -> [..., n])."""
    device = _lib.require_cuda(xq, w_packed)
    if xq.dtype != torch.int8:
        raise ValueError("gemm_i32 expects int8 activations")
    x2, ldq = _rows_view(xq)
    m, k = x2.shape
    _check_operands(k, w_packed, None, None, n, in_features)
    acc = torch.empty((m, n), dtype=torch.int32, device=device)
    if m and n:
        ws = _workspace(m, k, device)
        lib = _lib.load()
        _lib.check(lib.w8a8_gemm_i32(x2.data_ptr(), ldq, w_packed.data_ptr(), acc.data_ptr(), n,
                                     m, n, k, ws.data_ptr(), ws.numel(),
                                     _lib.stream_handle(device)), "w8a8_gemm_i32")
    return acc.reshape(*xq.shape[:-1], n)


def _out_cols(epilogue: int, n: int) -> int:
    return n // 2 if epilogue in (_lib.EPI_SILU_MUL, _lib.EPI_SILU_MUL_Q8) else n


def _default_out_dtype(epilogue: int, x_dtype: torch.dtype) -> torch.dtype:
    if epilogue == _lib.EPI_SILU_MUL_Q8:
        return torch.int8
    if epilogue == _lib.EPI_I32:
        return torch.int32
    if epilogue == _lib.EPI_DEQUANT_BF16_EXACT:
        return torch.bfloat16
    return x_dtype


def linear_dynamic(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                   bias: torch.Tensor | None, n: int, *, epilogue: int = _lib.EPI_DEQUANT,
                   out_dtype: torch.dtype | None = None, y_scale: float = 0.0,
                   inter_dtype: torch.dtype | None = None,
                   x_scale_out: torch.Tensor | None = None,
                   in_features: int | None = None) -> torch.Tensor:
    """Per-token dynamic A8 x per-output W8 linear with a fused epilogue."""
    device = _lib.require_cuda(x, w_packed, w_scale, bias)
    x2, ldx = _rows_view(x)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    if x_scale_out is not None and (x_scale_out.dtype != torch.float32
                                    or not x_scale_out.is_contiguous()
                                    or x_scale_out.numel() < m):
        raise ValueError("x_scale_out must be a contiguous float32 tensor with one value per row")
    if out_dtype is None:
        out_dtype = _default_out_dtype(epilogue, x.dtype)
    if inter_dtype is None:
        inter_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.float16
    cols = _out_cols(epilogue, n)
    y = torch.empty((m, cols), dtype=out_dtype, device=device)
    if m and n:
        lib = _lib.load()
        args = [x2.data_ptr(), _lib.dtype_code(x2.dtype), ldx, w_packed.data_ptr(),
                w_scale.data_ptr(), _lib.ptr(bias), epilogue, y.data_ptr(),
                _lib.dtype_code(out_dtype), cols, float(y_scale), _lib.dtype_code(inter_dtype),
                m, n, k, _lib.ptr(x_scale_out)]
        stream = _lib.stream_handle(device)
        # Decode shapes run fused and need no workspace; others report
        # ERR_WORKSPACE (before any launch) and are retried with one.
        rc = lib.w8a8_linear(*args, None, 0, stream)
        if rc == _lib.ERR_WORKSPACE:
            ws = _workspace(m, k, device)
            rc = lib.w8a8_linear(*args, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "w8a8_linear")
    return y.reshape(*x.shape[:-1], cols)


class ResidualOutput(NamedTuple):
    y: torch.Tensor                 # dtype(linear(x) + residual): the new residual stream
    ss_parts: torch.Tensor | None   # [rows, ceil(n/8)] binary32 RMSNorm chunk sums of y


def _residual_rows(residual: torch.Tensor, m: int, n: int,
                   dtype: torch.dtype) -> tuple[torch.Tensor, int]:
    if residual.dtype != dtype or residual.shape[-1] != n or residual.numel() != m * n:
        raise ValueError("residual must be [rows, n] rows of the output dtype")
    return _rows_view(residual)


def _residual_call(name: str, args: list, m: int, k: int, device, *, retry: bool) -> None:
    lib = _lib.load()
    stream = _lib.stream_handle(device)
    fn = getattr(lib, name)
    if retry:
        rc = fn(*args, None, 0, stream)
        if rc == _lib.ERR_WORKSPACE:
            ws = _workspace(m, k, device)
            rc = fn(*args, ws.data_ptr(), ws.numel(), stream)
    else:
        ws = _workspace(m, k, device)
        rc = fn(*args, ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, name)


def linear_residual(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                    bias: torch.Tensor | None, n: int, residual: torch.Tensor, *,
                    ss_parts: bool = True, in_features: int | None = None) -> ResidualOutput:
    """``residual + linear(x)`` in the activation dtype, the residual add of a
    decoder layer after its o_proj / down_proj (``residual_norm``,
    lightweight_runner.py:247-257, 552), folded into the dequant epilogue of
    the per-token dynamic W8A8 linear (``w8a8_linear_residual``).  With
    ``ss_parts`` the RMSNorm sums of squares of the result per 8 columns come
    back too, for :func:`rmsnorm_linear` on the same rows."""
    device = _lib.require_cuda(x, w_packed, w_scale, bias, residual)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the residual stream is float16 / bfloat16")
    x2, ldx = _rows_view(x)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    r2, ldr = _residual_rows(residual, m, n, x.dtype)
    y = torch.empty((m, n), dtype=x.dtype, device=device)
    nck = (n + 7) // 8
    parts = torch.empty((m, nck), dtype=torch.float32, device=device) if ss_parts else None
    if m and n:
        args = [x2.data_ptr(), _lib.dtype_code(x.dtype), ldx, w_packed.data_ptr(),
                w_scale.data_ptr(), _lib.ptr(bias), y.data_ptr(), _lib.dtype_code(x.dtype), n,
                r2.data_ptr(), ldr, _lib.ptr(parts), nck, m, n, k]
        # Decode shapes run fused and need no workspace (as linear_dynamic).
        _residual_call("w8a8_linear_residual", args, m, k, device, retry=True)
    return ResidualOutput(y.reshape(*x.shape[:-1], n), parts)


def linear_i8in_residual(xq: torch.Tensor, x_scale: torch.Tensor, w_packed: torch.Tensor,
                         w_scale: torch.Tensor, bias: torch.Tensor | None, n: int,
                         residual: torch.Tensor, *, ss_parts: bool = True,
                         in_features: int | None = None) -> ResidualOutput:
    """:func:`linear_residual` on int8 activations with per-row scales
    (``w8a8_linear_i8in_residual``); the output has the residual's dtype."""
    device = _lib.require_cuda(xq, x_scale, w_packed, w_scale, bias, residual)
    if xq.dtype != torch.int8:
        raise ValueError("linear_i8in_residual expects int8 activations")
    if residual.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the residual stream is float16 / bfloat16")
    x2, ldq = _rows_view(xq)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    s = x_scale.detach().to(dtype=torch.float32).reshape(-1).contiguous()
    if s.numel() != m:
        raise ValueError("x_scale must have one value per row")
    r2, ldr = _residual_rows(residual, m, n, residual.dtype)
    y = torch.empty((m, n), dtype=residual.dtype, device=device)
    nck = (n + 7) // 8
    parts = torch.empty((m, nck), dtype=torch.float32, device=device) if ss_parts else None
    if m and n:
        args = [x2.data_ptr(), ldq, s.data_ptr(), w_packed.data_ptr(), w_scale.data_ptr(),
                _lib.ptr(bias), y.data_ptr(), _lib.dtype_code(residual.dtype), n, r2.data_ptr(),
                ldr, _lib.ptr(parts), nck, m, n, k]
        _residual_call("w8a8_linear_i8in_residual", args, m, k, device, retry=False)
    return ResidualOutput(y.reshape(*xq.shape[:-1], n), parts)


def linear_i8in(xq: torch.Tensor, x_scale: torch.Tensor, w_packed: torch.Tensor,
                w_scale: torch.Tensor, bias: torch.Tensor | None, n: int, *,
                epilogue: int = _lib.EPI_DEQUANT, out_dtype: torch.dtype | None = None,
                y_scale: float = 0.0, inter_dtype: torch.dtype = torch.float16,
                in_features: int | None = None) -> torch.Tensor:
    """W8A8 linear on already-quantized activations with per-row scales."""
    device = _lib.require_cuda(xq, x_scale, w_packed, w_scale, bias)
    if xq.dtype != torch.int8:
        raise ValueError("linear_i8in expects int8 activations")
    if out_dtype is None:
        out_dtype = _default_out_dtype(epilogue, torch.float16)
    x2, ldq = _rows_view(xq)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    s = x_scale.detach().to(dtype=torch.float32).reshape(-1)
    if s.numel() == 1 and m != 1:
        s = s.expand(m)
    s = s.contiguous()
    if s.numel() != m:
        raise ValueError("x_scale must be per-tensor or one value per row")
    cols = _out_cols(epilogue, n)
    y = torch.empty((m, cols), dtype=out_dtype, device=device)
    if m and n:
        ws = _workspace(m, k, device)
        lib = _lib.load()
        _lib.check(lib.w8a8_linear_i8in(
            x2.data_ptr(), ldq, s.data_ptr(), w_packed.data_ptr(), w_scale.data_ptr(),
            _lib.ptr(bias), epilogue, y.data_ptr(), _lib.dtype_code(out_dtype), cols,
            float(y_scale), _lib.dtype_code(inter_dtype), m, n, k, ws.data_ptr(), ws.numel(),
            _lib.stream_handle(device)), "w8a8_linear_i8in")
    return y.reshape(*xq.shape[:-1], cols)


def linear_packed(xq_packed: torch.Tensor, x_scale: torch.Tensor, m: int, k: int,
                  w_packed: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None,
                  n: int, *, epilogue: int = _lib.EPI_DEQUANT,
                  out_dtype: torch.dtype | None = None, y_scale: float = 0.0,
                  inter_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """W8A8 linear on int8 activations already in the packed 16x64 tile
    layout of an [m, k] operand (``pack_rows`` output): the MFMA GEMM alone,
    no packing pass, no workspace."""
    device = _lib.require_cuda(xq_packed, x_scale, w_packed, w_scale, bias)
    if xq_packed.dtype != torch.int8 or xq_packed.numel() < packed_bytes(m, k):
        raise ValueError("xq_packed must hold the packed tiles of an [m, k] int8 operand")
    _check_operands(k, w_packed, w_scale, bias, n, k)
    s = x_scale.detach().to(dtype=torch.float32).reshape(-1).contiguous()
    if s.numel() != m:
        raise ValueError("x_scale must have one value per row")
    if out_dtype is None:
        out_dtype = _default_out_dtype(epilogue, torch.float16)
    cols = _out_cols(epilogue, n)
    y = torch.empty((m, cols), dtype=out_dtype, device=device)
    if m and n:
        lib = _lib.load()
        _lib.check(lib.w8a8_linear_packed(
            xq_packed.data_ptr(), s.data_ptr(), w_packed.data_ptr(), w_scale.data_ptr(),
            _lib.ptr(bias), epilogue, y.data_ptr(), _lib.dtype_code(out_dtype), cols,
            float(y_scale), _lib.dtype_code(inter_dtype), m, n, k,
            _lib.stream_handle(device)), "w8a8_linear_packed")
    return y


class TwoPhaseOutput(NamedTuple):
    h: torch.Tensor      # SiLU(g) * u, 16-bit [..., n/2]
    hq: torch.Tensor     # int8 [..., n/2], per-token dynamic quantization of h
    scale: torch.Tensor  # f32 [...], its per-row scales


def gateup_silu_mul_two_phase(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                              bias: torch.Tensor | None, n: int, *,
                              x_scale: torch.Tensor | None = None,
                              h_dtype: torch.dtype | None = None,
                              in_features: int | None = None) -> TwoPhaseOutput:
    """Packed gate/up with SiLU*mul, then the per-token dynamic int8
    quantization of h in two phases (``w8a8_gateup_silu_mul``): the epilogue
    leaves each row's |h|max per 16-row weight block in the workspace, and a
    second kernel quantizes h with ``scale_from_absmax`` of their max.  ``x``
    is 16/32-bit (quantized per token) or int8 with per-row ``x_scale``.
    ``hq`` and ``scale`` equal ``dynamic_per_token_activation_qdq``'s integer
    part of ``h`` (w8a8.py:106-115)."""
    device = _lib.require_cuda(x, w_packed, w_scale, bias, x_scale)
    x2, ldx = _rows_view(x)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    if n % 2:
        raise ValueError("packed gate/up needs an even number of rows")
    sx = None
    if x.dtype == torch.int8:
        if x_scale is None:
            raise ValueError("int8 activations need their per-row scales")
        sx = x_scale.detach().to(dtype=torch.float32).reshape(-1)
        if sx.numel() == 1 and m != 1:
            sx = sx.expand(m)
        sx = sx.contiguous()
        if sx.numel() != m:
            raise ValueError("x_scale must be per-tensor or one value per row")
    if h_dtype is None:
        h_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.float16
    cols = n // 2
    h = torch.empty((m, cols), dtype=h_dtype, device=device)
    hq = torch.empty((m, cols), dtype=torch.int8, device=device)
    hs = torch.empty((m,), dtype=torch.float32, device=device)
    if m and n:
        lib = _lib.load()
        ws = torch.empty((max(int(lib.w8a8_gateup_workspace_bytes(m, n, k)), 256),),
                         dtype=torch.uint8, device=device)
        _lib.check(lib.w8a8_gateup_silu_mul(
            x2.data_ptr(), _lib.dtype_code(x2.dtype), ldx, _lib.ptr(sx), w_packed.data_ptr(),
            w_scale.data_ptr(), _lib.ptr(bias), h.data_ptr(), _lib.dtype_code(h_dtype), cols,
            hq.data_ptr(), cols, hs.data_ptr(), m, n, k, ws.data_ptr(), ws.numel(),
            _lib.stream_handle(device)), "w8a8_gateup_silu_mul")
    lead = x.shape[:-1]
    return TwoPhaseOutput(h.reshape(*lead, cols), hq.reshape(*lead, cols), hs.reshape(lead))


class PrologueOutput(NamedTuple):
    q: torch.Tensor                  # int8 [..., K]
    scale: torch.Tensor              # f32 [...] per row (dynamic) or the static scale
    residual: torch.Tensor | None    # x + residual, when a residual was given
    rows: torch.Tensor | None        # the rows before quantization, when asked for


def prologue_quant(x: torch.Tensor, *, norm_weight: torch.Tensor | None = None,
                   eps: float = 1e-6, residual: torch.Tensor | None = None,
                   smooth: torch.Tensor | None = None,
                   static_scale: torch.Tensor | float | None = None,
                   return_rows: bool = False) -> PrologueOutput:
    """One pass per row of 16-bit ``x``: [x + residual] -> [RMSNorm with
    ``norm_weight``] -> [/ ``smooth``] -> int8 quantization (per-row dynamic
    scale, or ``static_scale``).  Each step follows its reference formula
    (lightweight_runner.py:239-257, w8a8.py:351-359, 94-115)."""
    device = _lib.require_cuda(x, norm_weight, residual, smooth)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the activation prologue takes float16 / bfloat16 rows")
    x2, ldx = _rows_view(x)
    m, k = x2.shape
    res2 = res_out = None
    ld_res = 0
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match the hidden states' shape and dtype")
        res2, ld_res = _rows_view(residual)
        res_out = torch.empty((m, k), dtype=x.dtype, device=device)
    w = None
    w_code = _lib.dtype_code(x.dtype)
    if norm_weight is not None:
        w = norm_weight.detach().reshape(-1)
        if w.numel() != k:
            raise ValueError("RMSNorm weight must have one value per hidden channel")
        if w.dtype not in (x.dtype, torch.float32):
            w = w.to(x.dtype)
        w = w.contiguous()
        w_code = _lib.dtype_code(w.dtype)
    sm = None
    if smooth is not None:
        sm = smooth.detach().reshape(-1).to(device=device, dtype=x.dtype).contiguous()
        if sm.numel() != k:
            raise ValueError("smoothing scales must have one value per input channel")
    st = None
    if static_scale is not None:
        st = torch.as_tensor(static_scale, dtype=torch.float32, device=device).reshape(1)
        if not bool(st[0] > 0):
            raise ValueError("quantization scale must be positive")
    q = torch.empty((m, k), dtype=torch.int8, device=device)
    scales = torch.empty((m,), dtype=torch.float32, device=device) if st is None else None
    rows = None
    if return_rows:
        rows_dtype = torch.float32 if (w is not None and w.dtype == torch.float32) else x.dtype
        rows = torch.empty((m, k), dtype=rows_dtype, device=device)
    if m and k:
        _lib.check(_lib.load().w8a8_prologue_quant(
            x2.data_ptr(), _lib.dtype_code(x.dtype), ldx, _lib.ptr(res2), ld_res,
            _lib.ptr(res_out), k, _lib.ptr(w), w_code, float(eps), _lib.ptr(sm), _lib.ptr(st),
            m, k, q.data_ptr(), k, _lib.ptr(scales), _lib.ptr(rows), k,
            _lib.stream_handle(device)), "w8a8_prologue_quant")
    lead = x.shape[:-1]
    return PrologueOutput(
        q.reshape(*lead, k),
        scales.reshape(lead) if scales is not None else st.reshape(()),
        None if res_out is None else res_out.reshape(x.shape),
        None if rows is None else rows.reshape(*lead, k))


class NormLinearOutput(NamedTuple):
    y: torch.Tensor                  # the linear's output
    residual: torch.Tensor | None    # hidden + residual, when a residual was given
    rows: torch.Tensor | None        # the normalized rows, when asked for


def rmsnorm_linear(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                   w_packed: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None,
                   n: int, *, residual: torch.Tensor | None = None,
                   epilogue: int = _lib.EPI_DEQUANT, out_dtype: torch.dtype | None = None,
                   y_scale: float = 0.0, return_rows: bool = False,
                   in_features: int | None = None,
                   ss_parts: torch.Tensor | None = None) -> NormLinearOutput:
    """``LightweightRMSNorm`` (lightweight_runner.py:239-257, with the
    residual add of ``residual_norm`` when ``residual`` is given) in front of a
    W8A8 linear with per-token dynamic quantization of the normalized rows:
    the W8A8 form of the reference's fused RMSNorm + packed QKV decode
    projection (paged_attention.py:163-234, 283-305).  A norm weight of x's
    dtype runs through ``w8a8_rmsnorm_linear`` (one kernel at decode shapes;
    otherwise the prologue writes the int8 rows in the product's own layout);
    a binary32 norm weight runs the activation prologue and the int8-in
    linear.

    ``ss_parts`` (no residual): the RMSNorm chunk sums of these very rows as
    :func:`linear_residual` returned them; the one-kernel decode route reads
    them instead of summing the rows in every workgroup
    (``w8a8_rmsnorm_linear_ss``, the same bits)."""
    device = _lib.require_cuda(x, norm_weight, w_packed, w_scale, bias, residual)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the activation prologue takes float16 / bfloat16 rows")
    x2, ldx = _rows_view(x)
    m, k = x2.shape
    _check_operands(k, w_packed, w_scale, bias, n, in_features)
    w = norm_weight.detach().reshape(-1)
    if w.numel() != k:
        raise ValueError("RMSNorm weight must have one value per hidden channel")
    if out_dtype is None:
        out_dtype = _default_out_dtype(epilogue, x.dtype)
    if w.dtype != x.dtype:
        # A binary32 weight promotes the normalized rows: prologue + int8 linear.
        pro = prologue_quant(x, norm_weight=norm_weight, eps=eps, residual=residual,
                             return_rows=return_rows)
        y = linear_i8in(pro.q, pro.scale.reshape(-1), w_packed, w_scale, bias, n,
                        epilogue=epilogue, out_dtype=out_dtype, y_scale=y_scale,
                        inter_dtype=x.dtype, in_features=in_features)
        return NormLinearOutput(y, pro.residual, pro.rows)
    w = w.contiguous()
    res2 = res_out = None
    ld_res = 0
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match the hidden states' shape and dtype")
        res2, ld_res = _rows_view(residual)
        res_out = torch.empty((m, k), dtype=x.dtype, device=device)
    rows = torch.empty((m, k), dtype=x.dtype, device=device) if return_rows else None
    cols = _out_cols(epilogue, n)
    y = torch.empty((m, cols), dtype=out_dtype, device=device)
    use_ss = ss_parts is not None and residual is None and not return_rows
    if use_ss:
        if (ss_parts.dtype != torch.float32 or ss_parts.dim() != 2
                or ss_parts.shape[0] != m or ss_parts.shape[1] < (k + 7) // 8
                or ss_parts.stride(1) != 1 or ss_parts.device != x.device):
            raise ValueError("ss_parts must be float32 [rows, >= ceil(K/8)] RMSNorm chunk sums")
    if m and n:
        lib = _lib.load()
        stream = _lib.stream_handle(device)
        if use_ss:
            name = "w8a8_rmsnorm_linear_ss"
            args = [x2.data_ptr(), _lib.dtype_code(x.dtype), ldx, ss_parts.data_ptr(),
                    ss_parts.stride(0), w.data_ptr(), float(eps), w_packed.data_ptr(),
                    w_scale.data_ptr(), _lib.ptr(bias), epilogue, y.data_ptr(),
                    _lib.dtype_code(out_dtype), cols, float(y_scale), _lib.dtype_code(x.dtype),
                    m, n, k, None]
        else:
            name = "w8a8_rmsnorm_linear"
            args = [x2.data_ptr(), _lib.dtype_code(x.dtype), ldx, _lib.ptr(res2), ld_res,
                    _lib.ptr(res_out), k, w.data_ptr(), float(eps), w_packed.data_ptr(),
                    w_scale.data_ptr(), _lib.ptr(bias), epilogue, y.data_ptr(),
                    _lib.dtype_code(out_dtype), cols, float(y_scale), _lib.dtype_code(x.dtype),
                    m, n, k, None, _lib.ptr(rows), k]
        fn = getattr(lib, name)
        rc = fn(*args, None, 0, stream)
        if rc == _lib.ERR_WORKSPACE:
            ws = _workspace(m, k, device)
            rc = fn(*args, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, name)
    lead = x.shape[:-1]
    return NormLinearOutput(y.reshape(*lead, cols),
                            None if res_out is None else res_out.reshape(x.shape),
                            None if rows is None else rows.reshape(x.shape))


def rmsnorm_quant(hidden_states: torch.Tensor, norm_weight: torch.Tensor, eps: float, *,
                  residual: torch.Tensor | None = None):
    """``LightweightRMSNorm`` (lightweight_runner.py:239-257) fused with the
    per-token int8 quantization of its output.  Returns ``(xq, s_x)``, or
    ``(summed, xq, s_x)`` with a residual, like ``residual_norm``."""
    out = prologue_quant(hidden_states, norm_weight=norm_weight, eps=eps, residual=residual)
    if residual is None:
        return out.q, out.scale
    return out.residual, out.q, out.scale


def smoothquant_activation_qdq(values: torch.Tensor, smoothing: torch.Tensor, *,
                               static_scale: torch.Tensor | float | None = None,
                               ) -> tuple[torch.Tensor, torch.Tensor]:
    """The SmoothQuant input hook's replacement (w8a8.py:351-362) on the GPU:
    ``values / smoothing`` then static or per-token dynamic QDQ.  Returns
    ``(qdq values, scale)``."""
    out = prologue_quant(values, smooth=smoothing, static_scale=static_scale)
    s = out.scale if static_scale is not None else out.scale.unsqueeze(-1)
    return (out.q.float() * s).to(values.dtype), s


# ------------------------------------------- reference-named contract functions
def quantize_symmetric(values: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``quantize_symmetric`` (w8a8.py:33-43) on the GPU.

    ``scale`` is one per-tensor value or one value per row of the last
    dimension (shape ``[..., 1]`` or ``[rows]``), the forms the contract uses.
    Non-positive scales raise ``ValueError`` (a host sync, as in the reference).
    """
    scale = torch.as_tensor(scale, device=values.device)
    if torch.any(scale <= 0):
        raise ValueError("quantization scale must be positive")
    return quant_rows_scaled(values, scale)


def scale_from_absmax(absmax: torch.Tensor) -> torch.Tensor:
    """``scale_from_absmax`` (w8a8.py:46-50): binary16-stored scale as f32."""
    _lib.require_cuda(absmax)
    raw = absmax.float().clamp_min(_F16_TINY) / CONTRACT.symmetric_max
    return raw.to(torch.float16).float().clamp_min(_F16_TINY)


def static_activation_scale(absmax, device: torch.device | str = "cuda") -> torch.Tensor:
    """``static_activation_scale`` (w8a8.py:94-98)."""
    value = torch.as_tensor(absmax, dtype=torch.float32, device=device)
    if value.numel() != 1:
        raise ValueError("static activation scale expects one tensor-wide absmax")
    return scale_from_absmax(value.reshape(()))


def static_activation_qdq(values: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``static_activation_qdq`` (w8a8.py:101-103)."""
    q = quantize_symmetric(values, scale)
    return (q.float() * scale.float().to(values.device)).to(values.dtype)


def dynamic_per_token_activation_qdq(values: torch.Tensor, *, axis: int = -1
                                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """``dynamic_per_token_activation_qdq`` (w8a8.py:106-115)."""
    if values.dim() == 0:
        raise ValueError("dynamic per-token quantization expects a tensor")
    moved = values.movedim(axis, -1)
    q, s = quant_rows(moved)
    scales = s.unsqueeze(-1)
    qdq = (q.float() * scales).to(values.dtype)
    return qdq.movedim(-1, axis), scales.movedim(-1, axis)


def per_output_weight_qdq(weight: torch.Tensor
                          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``per_output_weight_qdq`` (w8a8.py:53-62): (dequant, int8, f32 scales [N])."""
    if weight.dim() < 2:
        raise ValueError("weight must have at least two dimensions")
    rows = weight.detach().reshape(weight.shape[0], -1)
    q, scales = quant_rows(rows)
    deq = (q.float() * scales[:, None]).reshape_as(weight)
    return deq.to(weight.dtype), q.reshape_as(weight), scales


def groupwise_weight_qdq(weight: torch.Tensor, *, group_size: int = 128
                         ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``groupwise_weight_qdq`` (w8a8.py:65-91): one scale per row and group of
    ``group_size`` input columns (the last group may be shorter).  Returns
    (dequant, int8, f32 scales [rows, groups]).  Each group is a strided
    [rows, group] view quantized per row by the HIP kernel."""
    if weight.dim() < 2:
        raise ValueError("groupwise W8 expects at least two weight dimensions")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    device = _lib.require_cuda(weight)
    rows = weight.shape[0]
    flat = weight.detach().reshape(rows, -1)
    cols = flat.shape[1]
    groups = (cols + group_size - 1) // group_size
    q = torch.empty((rows, cols), dtype=torch.int8, device=device)
    deq = torch.empty((rows, cols), dtype=weight.dtype, device=device)
    scales = torch.empty((rows, groups), dtype=torch.float32, device=device)
    full = cols // group_size
    if full:
        body = flat[:, : full * group_size].float().reshape(rows * full, group_size)
        qb, sb = quant_rows(body)
        q[:, : full * group_size] = qb.reshape(rows, full * group_size)
        scales[:, :full] = sb.reshape(rows, full)
    if full < groups:
        qt, st = quant_rows(flat[:, full * group_size:].float())
        q[:, full * group_size:] = qt
        scales[:, full] = st
    per_col = scales.repeat_interleave(group_size, dim=1)[:, :cols]
    deq.copy_((q.float() * per_col).to(weight.dtype))
    return deq.reshape(weight.shape), q.reshape(weight.shape), scales


def tensor_error(reference: torch.Tensor, candidate: torch.Tensor) -> dict[str, float]:
    """``_tensor_error`` (w8a8.py:254-262)."""
    difference = candidate.float() - reference.float()
    denominator = reference.float().abs().clamp_min(1e-8)
    return {
        "rmse": float(difference.square().mean().sqrt().item()),
        "max_abs": float(difference.abs().max().item()),
        "mean_abs": float(difference.abs().mean().item()),
        "mean_relative_abs": float((difference.abs() / denominator).mean().item()),
    }


def compare_linear_bf16_qdq_integer(values: torch.Tensor, weight: torch.Tensor, *,
                                    activation_scale: torch.Tensor,
                                    bias: torch.Tensor | None = None) -> dict[str, Any]:
    """``compare_linear_bf16_qdq_integer`` (w8a8.py:142-214) with the integer
    path on the HIP kernels: native bf16, bf16 after QDQ, fp32 QDQ and the true
    int32 path, the same report keys and metrics.  The float paths use torch
    linears on the GPU in the reference's dtypes."""
    if values.shape[-1] != weight.shape[1] or weight.dim() != 2:
        raise ValueError("linear input/weight shapes do not match")
    if weight.shape[1] * CONTRACT.symmetric_max ** 2 >= 1 << 31:
        raise OverflowError("worst-case dot product exceeds signed INT32")
    device = _lib.require_cuda(values, weight)
    x = values.detach().float()
    w = weight.detach().float()
    b = None if bias is None else bias.detach().float().to(device)
    scale = torch.as_tensor(activation_scale, device=device).detach().float()
    qactivation = quantize_symmetric(x, scale)
    dequant_weight, _, _ = per_output_weight_qdq(w)
    dequant_activation = qactivation.float() * scale
    out_shape = (*values.shape[:-1], weight.shape[0])

    def linear(a, wt, bb):
        # 2-D products only (plain matrix multiplies, no batched bf16 calls).
        return torch.nn.functional.linear(a.reshape(-1, a.shape[-1]), wt, bb).reshape(out_shape)

    fp32_reference = linear(x, w, b)
    qdq_fp32 = linear(dequant_activation, dequant_weight, b)
    bf16 = torch.bfloat16
    bf16_reference = linear(x.to(bf16), w.to(bf16), None if b is None else b.to(bf16)).float()
    qdq_bf16 = linear(dequant_activation.to(bf16), dequant_weight.to(bf16),
                      None if b is None else b.to(bf16)).float()
    integer, accumulator = integer_linear_per_output(x, w, activation_scale=scale, bias=b)
    return {
        "source_device": str(values.device),
        "arithmetic_contract": {
            "activation_quantization": "symmetric_per_tensor_int8",
            "activation_scale_storage": CONTRACT.scale_storage,
            "weight_quantization": "symmetric_per_output_int8",
            "weight_scale_storage": CONTRACT.scale_storage,
            "accumulation": CONTRACT.accumulator,
            "dequantization_arithmetic": "float32",
            "bias_present": b is not None,
            "bias_application": CONTRACT.bias if b is not None else "none",
            "output_dtype": "float32",
        },
        "shape": {"input": list(values.shape), "weight": list(weight.shape),
                  "output": list(integer.shape)},
        "accumulator_dtype": str(accumulator.dtype),
        "accumulator_min": int(accumulator.min().item()),
        "accumulator_max": int(accumulator.max().item()),
        "worst_case_accumulator_bound": weight.shape[1] * CONTRACT.symmetric_max ** 2,
        "int32_safe": True,
        "metrics": {
            "bf16_vs_fp32": tensor_error(fp32_reference, bf16_reference),
            "qdq_bf16_vs_qdq_fp32": tensor_error(qdq_fp32, qdq_bf16),
            "integer_vs_qdq_fp32": tensor_error(qdq_fp32, integer),
            "integer_vs_qdq_bf16": tensor_error(qdq_bf16, integer),
            "integer_vs_fp32": tensor_error(fp32_reference, integer),
        },
    }


def integer_linear_per_output(values: torch.Tensor, weight: torch.Tensor, *,
                              activation_scale: torch.Tensor,
                              bias: torch.Tensor | None = None
                              ) -> tuple[torch.Tensor, torch.Tensor]:
    """GPU execution of ``integer_linear_per_output_reference`` (w8a8.py:118-139).

    Returns ``(out f32 [..., N], acc int32 [..., N])`` with the reference's
    arithmetic: int8 x int8 -> int32, then ``f32(acc) * s_x * s_w + bias``.
    """
    if values.shape[-1] != weight.shape[1] or weight.dim() != 2:
        raise ValueError("linear input/weight shapes do not match")
    device = _lib.require_cuda(values, weight)
    n = weight.shape[0]
    qa = quantize_symmetric(values, activation_scale)
    _, qw, sw = per_output_weight_qdq(weight)
    w_packed = pack_rows(qw)
    acc = gemm_i32(qa, w_packed, n)
    rows = qa.reshape(-1, qa.shape[-1]).shape[0]
    s = torch.as_tensor(activation_scale, device=device).float().reshape(-1)
    s = (s.expand(rows) if s.numel() == 1 else s).contiguous()
    b = None if bias is None else bias.detach().float().to(device).contiguous()
    out = linear_i8in(qa, s, w_packed, sw, b, n, out_dtype=torch.float32)
    return out, acc
