"""C ABI surface of libw8a8_gfx950.so, checked without a GPU: the library
loads, exports every entry point include/w8a8_gfx950.h declares, reports
sizes, and rejects bad arguments with status codes before any launch."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from nanopointllm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "w8a8_gfx950.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(w8a8_\w+)\s*\(", text, re.M)))


def test_header_declarations_are_exported():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) == len(_lib.EXPORTED_SYMBOLS) >= 16
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTED_SYMBOLS) == names


def test_sizes_and_version():
    lib = _lib.load()
    assert lib.w8a8_abi_version() == _lib.ABI_VERSION
    assert lib.w8a8_packed_bytes(12288, 4096) == 12288 * 4096
    assert lib.w8a8_packed_bytes(50, 100) == 64 * 128
    assert lib.w8a8_packed_bytes(-1, 4) == -1
    assert lib.w8a8_workspace_bytes(8, 4096) == 256 + 16 * 4096
    assert lib.w8a8_workspace_bytes(560, 11008) == 2304 + 560 * 11008
    assert lib.w8a8_status_string(_lib.ERR_WORKSPACE) == b"workspace missing or too small"


def test_invalid_arguments_return_status_without_launch():
    lib = _lib.load()
    # Never dereferenced: every call below fails validation before any launch
    # (none of them is a valid decode-path call that would run a kernel).
    fake = ctypes.c_void_p(0x1000)
    # negative shape
    assert lib.w8a8_quant_rows(fake, _lib.F16, -1, 4, 4, fake, 4, fake, None) == _lib.ERR_SHAPE
    # unsupported input dtype
    assert lib.w8a8_quant_rows(fake, _lib.I8, 1, 4, 4, fake, 4, fake, None) == _lib.ERR_DTYPE
    # null pointers
    assert lib.w8a8_quant_rows(None, _lib.F16, 1, 4, 4, fake, 4, fake, None) == _lib.ERR_NULL
    # leading dimension too small
    assert lib.w8a8_quant_rows(fake, _lib.F16, 2, 8, 4, fake, 8, fake, None) == _lib.ERR_SHAPE
    # K beyond the int32 accumulator bound (K * 127**2 >= 2**31)
    assert lib.w8a8_linear(fake, _lib.F16, 200000, fake, fake, None, _lib.EPI_DEQUANT, fake,
                           _lib.F16, 8, 0.0, _lib.F16, 1, 8, 133145, None, fake, 1 << 30,
                           None) == _lib.ERR_SHAPE
    # M or N beyond the kernels' int range
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_DEQUANT, fake,
                           _lib.F16, 1 << 31, 0.0, _lib.F16, 1, 1 << 31, 64, None, fake,
                           1 << 30, None) == _lib.ERR_SHAPE
    assert lib.w8a8_quant_rows(fake, _lib.F16, 1 << 31, 4, 4, fake, 4, fake,
                               None) == _lib.ERR_SHAPE
    # SiLU epilogue needs an even N and a 16-bit output
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_SILU_MUL, fake,
                           _lib.F32, 8, 0.0, _lib.F16, 1, 16, 64, None, fake, 1 << 20,
                           None) == _lib.ERR_DTYPE
    # int8 requant epilogue needs a positive static scale
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_SILU_MUL_Q8, fake,
                           _lib.I8, 8, 0.0, _lib.F16, 1, 16, 64, None, fake, 1 << 20,
                           None) == _lib.ERR_SHAPE
    # workspace too small (m = 17 is outside the workspace-free decode paths)
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_DEQUANT, fake,
                           _lib.F16, 16, 0.0, _lib.F16, 17, 16, 64, None, fake, 10,
                           None) == _lib.ERR_WORKSPACE
    # packed activations: misaligned, or a missing scale vector
    assert lib.w8a8_linear_packed(ctypes.c_void_p(0x1008), fake, fake, fake, None,
                                  _lib.EPI_DEQUANT, fake, _lib.F16, 16, 0.0, _lib.F16, 96, 16,
                                  64, None) == _lib.ERR_ALIGN
    assert lib.w8a8_linear_packed(fake, None, fake, fake, None, _lib.EPI_DEQUANT, fake,
                                  _lib.F16, 16, 0.0, _lib.F16, 96, 16, 64,
                                  None) == _lib.ERR_NULL
    assert lib.w8a8_linear_packed(fake, fake, fake, fake, None, _lib.EPI_REQUANT, fake,
                                  _lib.I8, 16, 0.0, _lib.F16, 96, 16, 64,
                                  None) == _lib.ERR_DTYPE
    # misaligned packed weights
    assert lib.w8a8_gemm_i32(fake, 64, ctypes.c_void_p(0x1001), fake, 16, 1, 16, 64, fake,
                             1 << 20, None) == _lib.ERR_ALIGN
    # interleaved packing needs an even row count
    assert lib.w8a8_pack_rows(fake, 3, 64, 64, _lib.ROWS_INTERLEAVE_HALVES, fake,
                              None) == _lib.ERR_SHAPE
    # empty problems are valid no-ops
    assert lib.w8a8_linear(None, _lib.F16, 64, None, None, None, _lib.EPI_DEQUANT, None,
                           _lib.F16, 16, 0.0, _lib.F16, 0, 16, 64, None, None, 0, None) == _lib.OK


def test_integer_epilogue_arguments_rejected_without_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    # the integer requant needs int8 activations with a static scale
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_REQUANT, fake,
                           _lib.I8, 16, 0.0, _lib.F16, 9, 16, 64, None, fake, 1 << 20,
                           None) == _lib.ERR_DTYPE
    assert lib.w8a8_linear_i8in(fake, 64, fake, fake, fake, None, _lib.EPI_REQUANT, fake,
                                _lib.I8, 16, 0.0, _lib.F16, 9, 16, 64, fake, 1 << 20,
                                None) == _lib.ERR_DTYPE
    # the single-rounding bf16 dequant has a bfloat16 output and no bias
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, fake, _lib.EPI_DEQUANT_BF16_EXACT,
                           fake, _lib.BF16, 16, 0.0, _lib.F16, 9, 16, 64, None, fake, 1 << 20,
                           None) == _lib.ERR_DTYPE
    assert lib.w8a8_linear(fake, _lib.F16, 64, fake, fake, None, _lib.EPI_DEQUANT_BF16_EXACT,
                           fake, _lib.F16, 16, 0.0, _lib.F16, 9, 16, 64, None, fake, 1 << 20,
                           None) == _lib.ERR_DTYPE
    # fused requant linear: null multiplier, short workspace, int8 output only
    assert lib.w8a8_linear_i8in_requant(fake, 64, fake, None, fake, None, fake, 16, 2, 16, 64,
                                        fake, 1 << 20, None) == _lib.ERR_NULL
    assert lib.w8a8_linear_i8in_requant(fake, 64, fake, fake, fake, None, fake, 16, 2, 16, 64,
                                        fake, 10, None) == _lib.ERR_WORKSPACE
    assert lib.w8a8_linear_i8in_requant(fake, 64, fake, fake, fake, ctypes.c_void_p(0x1002),
                                        fake, 16, 2, 16, 64, fake, 1 << 20,
                                        None) == _lib.ERR_ALIGN
    # elementwise epilogues
    assert lib.w8a8_requantize_i32(fake, 8, None, fake, fake, fake, 16, 2, 16,
                                   None) == _lib.ERR_SHAPE
    assert lib.w8a8_requantize_i32(fake, 16, None, fake, None, fake, 16, 2, 16,
                                   None) == _lib.ERR_NULL
    assert lib.w8a8_dequant_i32_bf16(fake, 16, fake, fake, ctypes.c_void_p(0x1001), 16, 2, 16,
                                     None) == _lib.ERR_ALIGN
    assert lib.w8a8_dequant_i32_bf16(None, 16, None, None, None, 16, 0, 16, None) == _lib.OK


def test_rmsnorm_linear_arguments_rejected_without_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)

    def call(*, x=fake, x_dtype=_lib.F16, residual=None, residual_out=None, norm=fake,
             eps=1e-6, epi=_lib.EPI_DEQUANT, bias=None, m=1, n=16, k=64, ldx=64, x_out=None):
        return lib.w8a8_rmsnorm_linear(x, x_dtype, ldx, residual, k, residual_out, k, norm, eps,
                                       fake, fake, bias, epi, fake, _lib.F16, n, 0.0, _lib.F16,
                                       m, n, k, None, x_out, k, None, 0, None)

    # rows of at most 32768 channels (the prologue holds a row in registers)
    assert call(k=32832, ldx=32832) == _lib.ERR_SHAPE
    # 16-bit rows only, and no integer requant epilogue
    assert call(x_dtype=_lib.F32) == _lib.ERR_DTYPE
    assert call(epi=_lib.EPI_REQUANT) == _lib.ERR_DTYPE
    # the RMSNorm weight, and residual_out with a residual, are required
    assert call(norm=None) == _lib.ERR_NULL
    assert call(residual=fake) == _lib.ERR_NULL
    assert call(x=None) == _lib.ERR_NULL
    # leading dimension, epsilon
    assert call(ldx=32) == _lib.ERR_SHAPE
    assert call(eps=-1.0) == _lib.ERR_SHAPE
    assert call(eps=float("nan")) == _lib.ERR_SHAPE
    # misaligned 16-bit operands
    assert call(norm=ctypes.c_void_p(0x1001)) == _lib.ERR_ALIGN
    assert call(x_out=ctypes.c_void_p(0x1003)) == _lib.ERR_ALIGN
    # empty problems are valid no-ops
    assert call(x=None, norm=None, m=0) == _lib.OK


def test_row_outputs_overlapping_inputs_are_rejected_without_launch():
    """residual_out and x_out may be the very rows of an input (in place);
    any other overlap, or the two outputs overlapping, is refused before any
    launch (a row-wise kernel would write rows another workgroup still reads)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    m, k = 2, 64
    row = k * 2                          # bytes of one binary16 row
    x, res = 0x100000, 0x200000

    def rl(residual=None, residual_out=None, x_out=None, ld_x_out=k):
        return lib.w8a8_rmsnorm_linear(ctypes.c_void_p(x), _lib.F16, k, _p(residual), k,
                                       _p(residual_out), k, fake, 1e-6, fake, fake, None,
                                       _lib.EPI_DEQUANT, fake, _lib.F16, 16, 0.0, _lib.F16,
                                       m, 16, k, None, _p(x_out), ld_x_out, None, 0, None)

    assert rl(x_out=x + row) == _lib.ERR_OVERLAP                # shifted by one row
    assert rl(x_out=x, ld_x_out=2 * k) == _lib.ERR_OVERLAP      # same base, other rows
    assert rl(residual=res, residual_out=res + 64) == _lib.ERR_OVERLAP
    assert rl(residual=res, residual_out=x + 2) == _lib.ERR_OVERLAP
    assert rl(residual=res, residual_out=0x300000, x_out=0x300000 + 2) == _lib.ERR_OVERLAP

    def pq(residual=None, residual_out=None, x_out=None, w_dtype=_lib.F16):
        return lib.w8a8_prologue_quant(ctypes.c_void_p(x), _lib.F16, k, _p(residual), k,
                                       _p(residual_out), k, fake, w_dtype, 1e-6, None, None,
                                       m, k, fake, k, fake, _p(x_out), k, None)

    assert pq(x_out=x + row) == _lib.ERR_OVERLAP
    assert pq(residual=res, residual_out=res + row) == _lib.ERR_OVERLAP
    # binary32 normalized rows written over the binary16 input rows: twice the
    # bytes per row, so not row for row.
    assert pq(x_out=x, w_dtype=_lib.F32) == _lib.ERR_OVERLAP
    assert lib.w8a8_status_string(_lib.ERR_OVERLAP) == (
        b"an output overlaps an input other than row for row")


def _p(addr):
    return None if addr is None else ctypes.c_void_p(addr)


def test_residual_add_arguments_rejected_without_launch():
    lib = _lib.load()
    fake, other = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x100000)
    parts = ctypes.c_void_p(0x200000)

    def lr(y_dtype=_lib.F16, res=other, ld_res=16, ss=parts, ld_ss=2, m=1, n=16, y=fake):
        return lib.w8a8_linear_residual(fake, _lib.F16, 64, fake, fake, None, y, y_dtype, 16,
                                        res, ld_res, ss, ld_ss, m, n, 64, fake, 1 << 20, None)
    # a 16-bit output only; the residual is required; leading dimensions
    assert lr(y_dtype=_lib.F32) == _lib.ERR_DTYPE
    assert lr(res=None) == _lib.ERR_NULL
    assert lr(ld_res=8) == _lib.ERR_SHAPE
    assert lr(ld_ss=1) == _lib.ERR_SHAPE
    # misaligned residual or sums
    assert lr(res=ctypes.c_void_p(0x100001)) == _lib.ERR_ALIGN
    assert lr(ss=ctypes.c_void_p(0x200002)) == _lib.ERR_ALIGN
    # y, residual and sums must not overlap
    assert lr(res=fake) == _lib.ERR_OVERLAP
    assert lr(ss=ctypes.c_void_p(0x1010)) == _lib.ERR_OVERLAP
    # empty problems are valid no-ops
    assert lr(m=0) == _lib.OK
    assert lib.w8a8_linear_i8in_residual(fake, 64, fake, fake, fake, None, fake, _lib.F32, 16,
                                         other, 16, parts, 2, 1, 16, 64, fake, 1 << 20,
                                         None) == _lib.ERR_DTYPE
    assert lib.w8a8_linear_i8in_residual(fake, 64, fake, fake, fake, None, fake, _lib.F16, 16,
                                         fake, 16, parts, 2, 1, 16, 64, fake, 1 << 20,
                                         None) == _lib.ERR_OVERLAP
    # RMSNorm on residual-stream rows: the sums cover every 8 columns of K
    assert lib.w8a8_rmsnorm_linear_ss(fake, _lib.F16, 64, parts, 7, fake, 1e-6, fake, fake, None,
                                      _lib.EPI_DEQUANT, other, _lib.F16, 16, 0.0, _lib.F16, 1,
                                      16, 64, None, fake, 1 << 20, None) == _lib.ERR_SHAPE
    assert lib.w8a8_rmsnorm_linear_ss(fake, _lib.F16, 64, ctypes.c_void_p(0x200002), 8, fake,
                                      1e-6, fake, fake, None, _lib.EPI_DEQUANT, other, _lib.F16,
                                      16, 0.0, _lib.F16, 1, 16, 64, None, fake, 1 << 20,
                                      None) == _lib.ERR_ALIGN


def test_dense_gemv_arguments_rejected_without_launch():
    lib = _lib.load()
    x, w, y, b = (ctypes.c_void_p(a) for a in (0x1000, 0x100000, 0x4000000, 0x8000000))

    def dg(x=x, ldx=64, w=w, ldw=64, bias=None, y=y, ldy=32, dtype=_lib.F16, m=8, n=32, k=64):
        return lib.w8a8_dense_gemv(x, ldx, w, ldw, bias, y, ldy, dtype, m, n, k, None)
    # 16-bit operands only; at most 16 rows; K a multiple of 8 up to 8192
    assert dg(dtype=_lib.F32) == _lib.ERR_DTYPE
    assert dg(dtype=_lib.I8) == _lib.ERR_DTYPE
    assert dg(m=17) == _lib.ERR_SHAPE
    assert dg(k=60, ldx=64, ldw=64) == _lib.ERR_SHAPE
    assert dg(k=8200, ldx=8200, ldw=8200) == _lib.ERR_SHAPE
    # leading dimensions: at least K (N for y), multiples of 8 for x and w
    assert dg(ldx=56) == _lib.ERR_SHAPE
    assert dg(ldw=68) == _lib.ERR_SHAPE
    assert dg(ldy=16) == _lib.ERR_SHAPE
    # null and misaligned operands
    assert dg(w=None) == _lib.ERR_NULL
    assert dg(x=ctypes.c_void_p(0x1008)) == _lib.ERR_ALIGN
    assert dg(bias=ctypes.c_void_p(0x8000001)) == _lib.ERR_ALIGN
    # y must not overlap x, w or the bias
    assert dg(y=ctypes.c_void_p(0x1040)) == _lib.ERR_OVERLAP
    assert dg(y=ctypes.c_void_p(0x100800)) == _lib.ERR_OVERLAP
    assert dg(bias=ctypes.c_void_p(0x4000010)) == _lib.ERR_OVERLAP
    # empty problems are valid no-ops
    assert dg(m=0) == _lib.OK
    assert dg(n=0) == _lib.OK


def test_dense_gemv_host_checks():
    import torch

    from nanopointllm_amd import lm_head

    x = torch.ones(2, 64, dtype=torch.float16)
    w = torch.ones(32, 64, dtype=torch.float16)
    assert not lm_head.dense_gemv_supported(x, w)  # CPU tensors
    with pytest.raises(RuntimeError, match="only on the GPU"):
        lm_head.dense_gemv(x, w)
    head = lm_head.DecodeLMHead(torch.nn.Linear(64, 32, bias=False).half())
    assert head.weight is head.linear.weight
    with pytest.raises(RuntimeError, match="only on the GPU"):
        head(x)


def test_status_errors_map_to_python_exceptions():
    with pytest.raises(ValueError, match="workspace"):
        _lib.check(_lib.ERR_WORKSPACE, "w8a8_linear")


def test_cpu_tensors_are_rejected_not_computed():
    import torch

    from nanopointllm_amd import w8a8

    with pytest.raises(RuntimeError, match="only on the GPU"):
        w8a8.quant_rows(torch.ones(2, 8, dtype=torch.float16))


def test_injection_requires_gpu_weights():
    import torch.nn as nn

    from nanopointllm_amd.inject import inject_w8a8

    model = nn.Module()
    model.model = nn.Module()
    layer = nn.Module()
    layer.mlp = nn.Module()
    layer.mlp.gate_proj = nn.Linear(8, 8)
    layer.mlp.up_proj = nn.Linear(8, 8)
    layer.mlp.down_proj = nn.Linear(8, 8)
    model.model.layers = nn.ModuleList([layer])
    with pytest.raises(RuntimeError, match="only on the GPU"):
        inject_w8a8(model)
