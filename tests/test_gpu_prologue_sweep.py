"""Seeded random sweep of the activation prologue (``w8a8.prologue_quant`` ->
``w8a8_prologue_quant``): [x + residual] -> [RMSNorm] -> [/ smooth] -> int8
(lightweight_runner.py:239-257; w8a8.py:351-359, 94-115), over its two
bodies (aligned rows with K % 8 == 0, and any other K or stride) and its
options: residual, norm weight of the rows' dtype or binary32 (which
promotes the rows to binary32), SmoothQuant divide, per-row dynamic scale or
a static one (binary16-representable or not), padded row strides.

Bars: without RMSNorm every step is an exactly rounded elementwise
operation, so the rows are bit-exact against the oracle; with it, within 2
ulps of the 16-bit dtype (binary32 sums of squares in another order) and
almost all bit-equal.  The summed residual, the scales and the int8
quantization of the kernel's own rows are bit-exact.
"""
from __future__ import annotations

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
        m = int(rng.integers(1, 9) if i % 2 else rng.integers(9, 301))
        k = int(rng.integers(1, 1537)) * 8 if rng.integers(0, 3) else int(rng.integers(5, 12289))
        cases.append(dict(
            i=i, m=m, k=k, dtype=["f16", "bf16"][int(rng.integers(0, 2))],
            res=bool(rng.integers(0, 2)), norm=["none", "16", "f32"][int(rng.integers(0, 3))],
            smooth=bool(rng.integers(0, 2)), static=["none", "f16", "any"][int(rng.integers(0, 3))],
            pad=int(rng.integers(0, 3)) * (8 if rng.integers(0, 2) else 3)))
    return cases


CASES = _cases(32, seed=20261204)


def _ids(c):
    return (f"{c['i']}-m{c['m']}-k{c['k']}-{c['dtype']}{'-res' if c['res'] else ''}-norm{c['norm']}"
            f"{'-smooth' if c['smooth'] else ''}-static{c['static']}-pad{c['pad']}")


@pytest.mark.parametrize("c", CASES, ids=[_ids(c) for c in CASES])
def test_prologue_random_case(cuda, c):
    from nanopointllm_amd import w8a8

    m, k, dtype, pad = c["m"], c["k"], c["dtype"], c["pad"]
    rng = np.random.default_rng(5000 + c["i"])
    tdt = TDT[dtype]
    xf = torch.from_numpy(rng.standard_normal((m, k + pad)).astype(np.float32) * 2).to(tdt)
    rf = torch.from_numpy(rng.standard_normal((m, k + pad)).astype(np.float32) * 0.5).to(tdt)
    x, r = xf[:, :k], rf[:, :k]                       # row stride k + pad
    w = torch.from_numpy(rng.random(k).astype(np.float32) + 0.5)
    if c["norm"] == "16":
        w = w.to(tdt)
    smooth = torch.from_numpy(np.exp(rng.random(k) * 2 - 1).astype(np.float32)).to(tdt)
    static = {"none": None, "f16": float(O.scale_from_absmax(np.float32(4.0))),
              "any": 0.0123456}[c["static"]]
    note(f"prologue sweep {_ids(c)}")
    out = w8a8.prologue_quant(
        xf.to(cuda)[:, :k], residual=rf.to(cuda)[:, :k] if c["res"] else None,
        norm_weight=None if c["norm"] == "none" else w.to(cuda), eps=1e-5,
        smooth=smooth.to(cuda) if c["smooth"] else None, static_scale=static, return_rows=True)

    y = x.float().numpy()
    if c["res"]:
        y = O.residual_add(y, r.float().numpy(), dtype)
        np.testing.assert_array_equal(out.residual.float().cpu().numpy(), y)
    f32_rows = c["norm"] == "f32"
    if c["norm"] != "none":
        y = O.rmsnorm(y, w.float().numpy(), 1e-5, dtype, weight_f32=f32_rows)
    if c["smooth"]:
        y = O.smooth_divide(y, smooth.float().numpy(), None if f32_rows else dtype)
    rows = out.rows.float().cpu().numpy()
    assert out.rows.dtype == (torch.float32 if f32_rows else tdt)
    if c["norm"] == "none":
        np.testing.assert_array_equal(rows, y)
    elif f32_rows:
        # a one-ulp flip of the 16-bit normalized value moves the row by at
        # most one 16-bit ulp, relatively (and the smooth divide keeps that)
        ulp16 = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7
        rel = np.abs(rows - y) / np.maximum(np.abs(y), 1e-30)
        assert rel.max() <= 1.01 * ulp16 and np.count_nonzero(rows != y) <= max(2, y.size // 1000)
    else:
        d = _ulps(rows, y, dtype)
        assert d.max() <= 2 and np.count_nonzero(d) <= max(2, d.size // 1000)
    if static is None:
        eq, es = O.dynamic_per_token_quant(rows)
        np.testing.assert_array_equal(out.scale.reshape(-1).cpu().numpy(), es[:, 0])
    else:
        eq = O.quantize_symmetric(rows, np.float32(static))
    np.testing.assert_array_equal(out.q.cpu().numpy(), eq)
