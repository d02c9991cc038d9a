"""Seeded random sweep of ``w8a8_rmsnorm_linear`` through the C ABI: residual
add + RMSNorm + per-token quantization + W8A8 linear (LightweightRMSNorm,
lightweight_runner.py:239-257; w8a8.py:106-139), over its routes: the fused
decode kernel (M <= 8, K <= 4096, enough weight per CU), the activation
prologue's vector body (K % 8 == 0, aligned rows) and its generic body
(other K), feeding the GEMV or the GEMM.

Each case draws M (1-8, 9-64 or 65-700), K (8-4096, a multiple of 8 or not),
padded row strides, an optional residual and bias, the 16-bit dtype and the
epilogue (int32, binary16 dequant, SiLU*mul, SiLU*mul + int8 requant; the
SiLU ones on binary16 rows, the dtype of the oracle's SiLU).  Bars: the
summed residual bit-exact against the oracle's; the normalized rows within 2
ulps of the oracle's RMSNorm and almost all bit-equal (binary32 sums of
squares in another order); the per-row scales and the int8 quantization of
the kernel's own rows bit-exact; the int32 accumulators exact; the dequant,
SiLU*mul and int8 h outputs equal to the oracle's on those rows.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

TDT = {"f16": torch.float16, "bf16": torch.bfloat16}


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _ulps(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(TDT[dtype]).view(torch.int16)
    u = torch.from_numpy(np.ascontiguousarray(b, np.float32)).to(TDT[dtype]).view(torch.int16)
    key = lambda i: torch.where(i < 0, -(i.int() & 0x7FFF), i.int())
    return (key(t) - key(u)).abs().numpy()


def _cases(count: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        regime = i % 3
        m = int(rng.integers(1, 9) if regime == 0 else
                rng.integers(9, 65) if regime == 1 else rng.integers(65, 701))
        k = int(rng.integers(1, 513)) * 8 if rng.integers(0, 3) else int(rng.integers(8, 4097))
        dtype = ["f16", "bf16"][int(rng.integers(0, 2))]
        epi = ["i32", "f16", "silu", "q8"][int(rng.integers(0, 4))]
        if dtype == "bf16" and epi in ("silu", "q8"):
            epi = "f16"
        n = 2 * int(rng.integers(8, 1501))
        if regime == 0 and rng.integers(0, 2):
            n = [12288, 16384, 22016][int(rng.integers(0, 3))]   # enough weight for the fused route
        pad = 8 * int(rng.integers(0, 3))
        cases.append((i, m, n, k, dtype, epi, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), pad))
    # Decode shapes with enough weight per CU for the fused kernel.
    for j, (m, n, k, dtype, epi, res) in enumerate([
            (8, 22016, 4096, "f16", "q8", True), (4, 12288, 4096, "bf16", "f16", False),
            (8, 12288, 4096, "f16", "silu", True), (1, 16384, 2048, "f16", "i32", True),
            (6, 22016, 3072, "f16", "silu", True)]):
        cases.append((count + j, m, n, k, dtype, epi, res, True, 8))
    return cases


CASES = _cases(36, seed=20261203)


def _ids(c):
    i, m, n, k, dtype, epi, res, bias, pad = c
    return f"{i}-m{m}-n{n}-k{k}-{dtype}-{epi}{'-res' if res else ''}{'-bias' if bias else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rmsnorm_linear_random_case(cuda, case):
    from nanopointllm_amd import _lib, w8a8

    i, m, n, k, dtype, epi, with_res, with_bias, pad = case
    rng = np.random.default_rng(4000 + i)
    tdt = TDT[dtype]
    x = torch.from_numpy(rng.standard_normal((m, k + pad)).astype(np.float32) * 2).to(tdt)
    x[:, rng.integers(0, k, size=max(1, k // 300))] *= 20
    r = torch.from_numpy(rng.standard_normal((m, k + pad)).astype(np.float32) * 0.5).to(tdt)
    nw = torch.from_numpy(rng.random(k).astype(np.float32) + 0.5).to(tdt)
    qw = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05 + 1e-3).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) if with_bias and epi != "i32" else None
    h_scale = float(O.scale_from_absmax(np.float32(3.0)))

    cols = n // 2 if epi in ("silu", "q8") else n
    code = {"i32": _lib.EPI_I32, "f16": _lib.EPI_DEQUANT, "silu": _lib.EPI_SILU_MUL,
            "q8": _lib.EPI_SILU_MUL_Q8}[epi]
    y_dtype = {"i32": torch.int32, "f16": torch.float16, "silu": torch.float16,
               "q8": torch.int8}[epi]
    xd, rd, nwd = x.to(cuda), r.to(cuda), nw.to(cuda)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swd = torch.from_numpy(sw).to(cuda)
    bd = None if bias is None else torch.from_numpy(bias).to(cuda)
    y = torch.empty(m, cols, dtype=y_dtype, device=cuda)
    rows = torch.empty(m, k, dtype=tdt, device=cuda)
    res_out = torch.empty(m, k, dtype=tdt, device=cuda)
    sx = torch.empty(m, dtype=torch.float32, device=cuda)
    lib = _lib.load()
    # Poisoned: the int8 rows' pad columns (K up to the next multiple of 64)
    # must be written as zeros by the call itself.
    ws = torch.full((lib.w8a8_workspace_bytes(m, k),), 0x5A, dtype=torch.uint8, device=cuda)
    ptr = lambda t: None if t is None else t.data_ptr()
    note(f"rmsnorm_linear sweep {_ids(case)}")
    rc = lib.w8a8_rmsnorm_linear(
        xd.data_ptr(), _lib.dtype_code(tdt), k + pad, rd.data_ptr() if with_res else None,
        k + pad, res_out.data_ptr() if with_res else None, k, nwd.data_ptr(),
        ctypes.c_float(1e-6), wp.data_ptr(), swd.data_ptr(), ptr(bd), code, y.data_ptr(),
        _lib.dtype_code(y_dtype), cols, ctypes.c_float(h_scale if epi == "q8" else 0.0),
        _lib.dtype_code(tdt), m, n, k, sx.data_ptr(), rows.data_ptr(), k, ws.data_ptr(),
        ws.numel(), _lib.stream_handle(cuda))
    assert rc == _lib.OK, lib.w8a8_status_string(rc)

    xs = x.float().numpy()[:, :k]
    summed = xs
    if with_res:
        summed = O.residual_add(xs, r.float().numpy()[:, :k], dtype)
        np.testing.assert_array_equal(res_out.float().cpu().numpy(), summed)
    got_rows = rows.float().cpu().numpy()
    d = _ulps(got_rows, O.rmsnorm(summed, nw.float().numpy(), 1e-6, dtype), dtype)
    assert d.max() <= 2 and np.count_nonzero(d) <= max(2, d.size // 1000)
    xq, es = O.dynamic_per_token_quant(got_rows)
    np.testing.assert_array_equal(sx.cpu().numpy(), es[:, 0])
    acc = O.int32_matmul_f64(xq, qw)
    got = y.cpu().numpy()
    if epi == "i32":
        np.testing.assert_array_equal(got, acc)
    elif epi == "f16":
        np.testing.assert_array_equal(got, O.dequant_epilogue(acc, es, sw, bias).astype(np.float16))
    else:
        eh = O.gateup_silu_mul_from_acc(acc, es, sw, bias, layout="interleave")
        if epi == "silu":
            np.testing.assert_array_equal(got, eh)
        else:
            np.testing.assert_array_equal(got, O.quantize_symmetric(eh, h_scale))
