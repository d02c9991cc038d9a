"""The LM head at decode batches (``w8a8_dense_gemv``): the reference's
``F.linear`` of up to 16 final-norm rows with the 16-bit ``lm_head`` weight
(``_decode_linear_rows`` / ``_decode_staged_linear``,
lightweight_runner.py:38-43, 96-99, 676-681).

Floating point, so the bar is a tolerance, written here: every output within
one unit in the last place of the output type (binary16: 2^(e-10),
bfloat16: 2^(e-7), e = floor(log2 |ref|), subnormal spacing at the bottom)
of the float64 product of the same 16-bit inputs, plus the binary32
accumulation bound K * 2^-24 * sum |x w|.  A transposed operand, a wrong row
or column mapping or a dropped K range misses it by orders of magnitude.
Also: deterministic, a row's values independent of the batch, overflow to
inf and NaN confined to its row, graph replays equal to eager, and the
``DecodeLMHead`` wrapper's routing.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nanopointllm_amd.lm_head import DecodeLMHead, dense_gemv, dense_gemv_supported

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _ulp(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    mant, tiny = (10, 2.0 ** -24) if dtype == torch.float16 else (7, 2.0 ** -133)
    a = np.abs(ref)
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.maximum(2.0 ** (e - mant), tiny)


def _check(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> None:
    xs = x.reshape(-1, x.shape[-1]).double().cpu().numpy()
    ws = w.double().cpu().numpy()
    ref = xs @ ws.T
    mag = np.abs(xs) @ np.abs(ws).T
    if b is not None:
        ref = ref + b.double().cpu().numpy()
    got = y.reshape(ref.shape).double().cpu().numpy()
    k = xs.shape[1]
    tol = _ulp(ref, y.dtype) + k * 2.0 ** -24 * mag
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} outputs off; worst {err[bad].max()} "
                           f"at {np.argwhere(bad)[0].tolist()}")


def _operands(m, n, k, dtype, seed, device, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(dtype).to(device)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype).to(device)
    b = (torch.randn(n, generator=g) * 0.1).to(dtype).to(device) if bias else None
    return x, w, b


SHAPES = [
    # LLaMA-7B's LM head (32003 x 4096) at decode batches
    (1, 32003, 4096), (8, 32003, 4096), (16, 32003, 4096),
    # 2-7 rows; fewer blocks than CUs; one block; one row of weights
    (3, 4096, 4096), (5, 17, 4096), (2, 16, 1024), (1, 1, 64),
    # several blocks per workgroup
    (4, 16 * 256 * 3 + 5, 512),
    # K off the 64-column step, the shortest K, and the longer-row variant
    (8, 1000, 4104), (8, 300, 40), (2, 100, 8), (8, 2000, 5120), (4, 777, 8192),
    # 9-16 rows (a second group of x rows), short and long K
    (9, 4096, 4096), (12, 1000, 4104), (13, 33, 8192), (16, 300, 40),
]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_dense_gemv_matches_float64_product(cuda, m, n, k):
    note(f"dense_gemv f16 m={m} n={n} k={k}")
    x, w, _ = _operands(m, n, k, torch.float16, 1000 + m + n + k, cuda)
    y = dense_gemv(x, w)
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == torch.float16
    _check(y, x, w, None)


@pytest.mark.parametrize("m,n,k", [(8, 32003, 4096), (1, 4100, 4096), (16, 515, 5120)])
def test_dense_gemv_bf16_with_bias(cuda, m, n, k):
    note(f"dense_gemv bf16+bias m={m} n={n} k={k}")
    x, w, b = _operands(m, n, k, torch.bfloat16, 2000 + m + k, cuda, bias=True)
    y = dense_gemv(x, w, b)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    _check(y, x, w, b)


def test_dense_gemv_f16_bias_and_torch(cuda):
    m, n, k = 8, 32003, 4096
    note(f"dense_gemv f16+bias vs F.linear m={m} n={n} k={k}")
    x, w, b = _operands(m, n, k, torch.float16, 7, cuda, bias=True)
    y = dense_gemv(x, w, b)
    _check(y, x, w, b)
    # the reference's F.linear on the same box: both within an ulp of the
    # float64 product, so within two of each other
    t = F.linear(x, w, b)
    torch.cuda.synchronize()
    ref = (x.double() @ w.double().T + b.double()).cpu().numpy()
    assert (np.abs(y.double().cpu().numpy() - t.double().cpu().numpy())
            <= 2 * _ulp(ref, torch.float16) + k * 2.0 ** -23 *
            (x.double().abs() @ w.double().abs().T).cpu().numpy()).all()


def test_dense_gemv_rows_independent_and_deterministic(cuda):
    m, n, k = 16, 4099, 4096
    note(f"dense_gemv batch independence m={m} n={n} k={k}")
    x, w, _ = _operands(m, n, k, torch.float16, 11, cuda)
    y = dense_gemv(x, w)
    assert torch.equal(dense_gemv(x, w), y)
    # single rows and 8-row batches (one group of x rows) against 16 (two)
    for r in (0, 7, 8, 15):
        assert torch.equal(dense_gemv(x[r:r + 1], w), y[r:r + 1])
    assert torch.equal(dense_gemv(x[3:11], w), y[3:11])
    assert torch.equal(dense_gemv(x[5:14], w), y[5:14])


def test_dense_gemv_strided_rows_and_3d_input(cuda):
    m, n, k = 6, 2048, 1024
    note(f"dense_gemv strided rows m={m} n={n} k={k}")
    g = torch.Generator().manual_seed(5)
    big = torch.randn(m, k + 64, generator=g).half().to(cuda)
    x = big[:, :k]  # leading dimension k + 64
    w = (torch.randn(n, k, generator=g) * 0.02).half().to(cuda)
    y = dense_gemv(x, w)
    assert torch.equal(y, dense_gemv(x.contiguous(), w))
    _check(y, x, w, None)
    y3 = dense_gemv(x.contiguous().view(1, m, k), w)
    assert y3.shape == (1, m, n) and torch.equal(y3[0], y)


def test_dense_gemv_special_values(cuda):
    m, n, k = 4, 64, 256
    note(f"dense_gemv inf/nan m={m} n={n} k={k}")
    x = torch.zeros(m, k, dtype=torch.float16)
    w = torch.ones(n, k, dtype=torch.float16)
    x[0] = 1.0            # row 0: 256 per output
    x[1] = 300.0          # row 1: 76800 > 65504 -> inf
    x[2, 5] = float("nan")  # row 2: NaN
    x[3] = -1.0 / 256     # row 3: -1
    y = dense_gemv(x.to(cuda), w.to(cuda)).cpu()
    assert torch.equal(y[0], torch.full((n,), 256.0, dtype=torch.float16))
    assert torch.isinf(y[1]).all() and (y[1] > 0).all()
    assert torch.isnan(y[2]).all()
    assert torch.equal(y[3], torch.full((n,), -1.0, dtype=torch.float16))


def test_dense_gemv_graph_replays_equal_eager(cuda):
    m, n, k = 8, 32003, 4096
    note(f"dense_gemv graph m={m} n={n} k={k}")
    x, w, _ = _operands(m, n, k, torch.float16, 21, cuda)
    eager = dense_gemv(x, w)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dense_gemv(x, w)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = dense_gemv(x, w)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        x.mul_(1.0)  # eager work between replays


def test_decode_lm_head_routes(cuda):
    k, n = 512, 1000
    note(f"DecodeLMHead routing n={n} k={k}")
    lin = torch.nn.Linear(k, n, bias=False).half().to(cuda)
    head = DecodeLMHead(lin)
    g = torch.Generator().manual_seed(3)
    rows = torch.randn(1, 16, k, generator=g).half().to(cuda)
    assert dense_gemv_supported(rows, lin.weight)
    assert torch.equal(head(rows), dense_gemv(rows, lin.weight))
    many = torch.randn(17, k, generator=g).half().to(cuda)
    assert not dense_gemv_supported(many, lin.weight)
    assert torch.equal(head(many), F.linear(many, lin.weight))
    with pytest.raises(ValueError, match="at most 16 rows"):
        dense_gemv(many, lin.weight)
