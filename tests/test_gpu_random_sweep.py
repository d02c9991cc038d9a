"""Seeded random sweep of ``w8a8_linear`` through the C ABI, over its three
routes (the fused decode kernel, the GEMV behind a quantization launch, the
MFMA GEMM) and its epilogues, against the oracle on the same inputs.

Each case draws M from one regime (1-16, 17-64 or 65-700), an even N, a K
from 1 to 4200 (most not a multiple of 64), the activation dtype, an optional
bias and a padded row stride.  Bars, as everywhere: the per-row scales and
int32 accumulators bit-exact against ``w8a8_linear_dynamic``
(w8a8.py:106-139); binary16 / bfloat16 / binary32 dequant outputs bit-equal
to the oracle's binary32 result rounded once; the packed gate/up SiLU*mul
output equal to the oracle's (torch's ``F.silu`` on the binary16 gate and
up, lightweight_runner.py:358); the single-rounding bf16 dequant equal to
``dequantize_int32_to_bf16`` (gtsu_cycle/bf16_dequant.py:47-94).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _cases(count: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        regime = i % 3
        m = int(rng.integers(1, 17) if regime == 0 else
                rng.integers(17, 65) if regime == 1 else rng.integers(65, 701))
        epi = ["i32", "f16", "bf16", "f32", "silu", "bf16x"][int(rng.integers(0, 6))]
        if epi == "bf16x" and m * 64 > 4096:
            epi = "bf16"          # the scalar oracle of the bf16 rounding is slow
        n = 2 * int(rng.integers(8, 3001))
        if epi == "bf16x":
            n = 2 * int(rng.integers(8, max(9, 2048 // m)))
        k = int(rng.integers(1, 4201))
        x_dtype = ["f16", "bf16", "f32"][int(rng.integers(0, 3))]
        if epi == "silu":
            x_dtype = "f16"       # the SiLU oracle rounds through binary16
        pad = 8 * int(rng.integers(0, 3))
        bias = bool(rng.integers(0, 2)) and epi != "bf16x"
        cases.append((i, m, n, k, x_dtype, epi, bias, pad))
    # Decode shapes large enough for the fused kernel (weights per CU >= 64 KiB).
    for j, (m, n, k) in enumerate([(3, 12288, 4096), (8, 22016, 4096), (5, 32768, 1000),
                                   (16, 24576, 4096)]):
        for epi, x_dtype in (("f16", "bf16"), ("silu", "f16")):
            cases.append((count + 2 * j + (epi == "silu"), m, n, k, x_dtype, epi, True, 8))
    return cases


CASES = _cases(36, seed=20261202)


def _ids(c):
    i, m, n, k, xd, epi, bias, pad = c
    return f"{i}-m{m}-n{n}-k{k}-{xd}-{epi}{'-bias' if bias else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_w8a8_linear_random_case(cuda, case):
    from nanopointllm_amd import _lib, w8a8

    i, m, n, k, x_dtype, epi, with_bias, pad = case
    rng = np.random.default_rng(1000 + i)
    x = rng.standard_normal((m, k + pad)).astype(np.float32) * 2.0
    x[:, rng.integers(0, k, size=max(1, k // 200))] *= 20.0
    xt = torch.from_numpy(x).to(_DTYPES[x_dtype])
    xv = xt.float().numpy()[:, :k]            # the values the kernels see
    qw = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05 + 1e-3).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) if with_bias else None

    silu = epi == "silu"
    code = {"i32": _lib.EPI_I32, "silu": _lib.EPI_SILU_MUL,
            "bf16x": _lib.EPI_DEQUANT_BF16_EXACT}.get(epi, _lib.EPI_DEQUANT)
    y_dtype = {"i32": torch.int32, "f16": torch.float16, "bf16": torch.bfloat16,
               "f32": torch.float32, "silu": torch.float16, "bf16x": torch.bfloat16}[epi]
    cols = n // 2 if silu else n
    lib = _lib.load()
    xd = xt.to(cuda)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt = torch.from_numpy(sw).to(cuda)
    bt = None if bias is None else torch.from_numpy(bias).to(cuda)
    y = torch.empty(m, cols, dtype=y_dtype, device=cuda)
    sx = torch.full((m,), -1.0, device=cuda)
    ws = torch.empty(lib.w8a8_workspace_bytes(m, k), dtype=torch.uint8, device=cuda)
    note(f"random sweep {_ids(case)}")

    def call(out, workspace):
        return lib.w8a8_linear(xd.data_ptr(), _lib.dtype_code(xt.dtype), k + pad, wp.data_ptr(),
                               swt.data_ptr(), None if bt is None else bt.data_ptr(), code,
                               out.data_ptr(), _lib.dtype_code(y_dtype), cols, 0.0, _lib.F16,
                               m, n, k, sx.data_ptr(),
                               None if workspace is None else workspace.data_ptr(),
                               0 if workspace is None else workspace.numel(),
                               _lib.stream_handle(cuda))

    rc = call(y, ws)
    assert rc == _lib.OK, lib.w8a8_status_string(rc)
    if i >= len(CASES) - 8:
        # The decode shapes sized for the fused kernel: it runs without a
        # workspace (every other route refuses a null one before launching).
        y2 = torch.empty_like(y)
        assert call(y2, None) == _lib.OK
        assert torch.equal(y2, y)

    exp, eacc, _, esx = O.w8a8_linear_dynamic(xv, qw, sw, bias)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    got = y.cpu()
    if epi == "i32":
        np.testing.assert_array_equal(got.numpy(), eacc)
    elif epi == "f16":
        np.testing.assert_array_equal(got.numpy(), exp.astype(np.float16))
    elif epi == "bf16":
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16),
                                      O.f32_to_bf16_bits(exp))
    elif epi == "f32":
        np.testing.assert_array_equal(got.numpy(), exp)
    elif epi == "silu":
        # Adjacent (even, odd) weight rows are a (gate, up) pair: the layout
        # pack_gateup_rows(..., "interleave") gives.
        eh = O.gateup_silu_mul_from_acc(eacc, esx, sw, bias, layout="interleave")
        np.testing.assert_array_equal(got.numpy(), eh)
    else:
        sa_bits = esx[:, 0].astype(np.float16).view(np.uint16)
        sw_bits = sw.astype(np.float16).view(np.uint16)
        want = np.array([[O.dequantize_int32_to_bf16(int(eacc[r, c]), int(sa_bits[r]),
                                                     int(sw_bits[c])) for c in range(n)]
                         for r in range(m)], dtype=np.uint16)
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), want)
