"""The residual stream of a decoder layer on the W8A8 kernels: the residual
add after o_proj / down_proj (``residual_norm``, lightweight_runner.py:247-257,
552) folded into the dequant epilogue of the linear, the RMSNorm sums of
squares that epilogue writes per 8 columns, and the RMSNorm + projection
launch that reads them (``w8a8_linear_residual``,
``w8a8_linear_i8in_residual``, ``w8a8_rmsnorm_linear_ss``).

Bars: the summed rows bit-equal to the oracle's per-token W8A8 linear rounded
to the activation dtype and added to the residual in that dtype (one
rounding, as torch adds two 16-bit tensors); the chunk sums bit-equal to the
order of the norm kernels (per chunk from +0 in column order, each square
rounded to binary32, one rounding per add); and the norm launch on those sums
bit-equal to the same launch summing the rows itself, on every route: the
fused decode kernels (M <= 4 with quantization inside, M = 8 and 12 after a
quantization launch on gemv_kernel, the int8-x stream at K > 8192), the
GEMV past 16 rows, and the GEMM with the add as a pass after it; N off the
16- and 8-column grids.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _weights(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    rng = np.random.default_rng(seed)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    return wq, sw, bias


def _chunk_sums(y: np.ndarray) -> np.ndarray:
    """Per row and 8-column chunk: fl(... fl(y0^2) + ... + y7^2) in binary32,
    columns past the row counting 0."""
    m, n = y.shape
    nck = -(-n // 8)
    sq = np.zeros((m, nck * 8), np.float32)
    sq[:, :n] = y.astype(np.float32) * y.astype(np.float32)
    sq = sq.reshape(m, nck, 8)
    s = np.zeros((m, nck), np.float32)
    for j in range(8):
        s = (s + sq[:, :, j]).astype(np.float32)
    return s


def _expected(xq, sx, wq, sw, bias, res16, dtype):
    acc = O.int32_matmul_f64(xq, wq)
    y32 = O.dequant_epilogue(acc, sx, sw, bias)
    y = torch.from_numpy(y32).to(dtype) + res16
    return y


@pytest.mark.parametrize("m,n,k,dtype", [
    (1, 4096, 4096, torch.float16), (4, 4096, 4096, torch.float16),
    (8, 4096, 4096, torch.float16), (12, 4096, 4096, torch.float16),
    (40, 4096, 4096, torch.float16), (100, 4096, 4096, torch.float16),
    (8, 1004, 1000, torch.float16), (100, 1004, 1000, torch.float16),
    (8, 4096, 4096, torch.bfloat16), (100, 4100, 700, torch.bfloat16),
    (5, 4096, 11008, torch.float16), (2, 300, 11264, torch.bfloat16),
    (7, 4096, 4104, torch.float16), (11, 4096, 4096, torch.float16),
    (16, 4096, 4096, torch.bfloat16),
])
def test_linear_residual_matches_the_oracle(cuda, m, n, k, dtype):
    from nanopointllm_amd import w8a8

    wq, sw, bias = _weights(n, k, seed=m + n + k)
    g = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn(m, k, generator=g) * 2).to(dtype)
    res = torch.randn(m, n, generator=g).to(dtype)
    note(f"linear_residual m={m} n={n} k={k} {dtype}")
    xq, sx = O.dynamic_per_token_quant(x.float().numpy())
    want = _expected(xq, sx, wq.numpy(), sw, bias, res, dtype)
    wp = w8a8.pack_rows(wq.to(cuda))
    swt, bt = torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda)
    out = w8a8.linear_residual(x.to(cuda), wp, swt, bt, n, res.to(cuda))
    assert out.y.dtype == dtype
    assert torch.equal(out.y.cpu(), want)
    np.testing.assert_array_equal(out.ss_parts.cpu().numpy(), _chunk_sums(want.float().numpy()))
    # The sums are optional; the rows are the same without them.
    plain = w8a8.linear_residual(x.to(cuda), wp, swt, bt, n, res.to(cuda), ss_parts=False)
    assert plain.ss_parts is None and torch.equal(plain.y, out.y)


@pytest.mark.parametrize("m,n,k", [(3, 4096, 11008), (8, 4096, 11008), (20, 4096, 11008),
                                   (70, 4096, 11008), (8, 4096, 4096)])
def test_linear_i8in_residual_matches_the_oracle(cuda, m, n, k):
    from nanopointllm_amd import w8a8

    wq, sw, _ = _weights(n, k, seed=5 + m + k)
    g = torch.Generator().manual_seed(m + 3)
    xq = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    sx = O.scale_from_absmax(np.abs(np.random.default_rng(m).standard_normal((m, 1))) * 3
                             ).astype(np.float32)
    res = torch.randn(m, n, generator=g).half()
    note(f"linear_i8in_residual m={m} n={n} k={k}")
    want = _expected(xq.numpy(), sx, wq.numpy(), sw, None, res, torch.float16)
    wp = w8a8.pack_rows(wq.to(cuda))
    out = w8a8.linear_i8in_residual(xq.to(cuda), torch.from_numpy(sx).to(cuda), wp,
                                    torch.from_numpy(sw).to(cuda), None, n, res.to(cuda))
    assert torch.equal(out.y.cpu(), want)
    np.testing.assert_array_equal(out.ss_parts.cpu().numpy(), _chunk_sums(want.float().numpy()))


@pytest.mark.parametrize("m", [1, 3, 5, 8, 12])
@pytest.mark.parametrize("proj", ["qkv", "gateup"])
def test_rmsnorm_on_the_sums_equals_rmsnorm_on_the_rows(cuda, m, proj):
    """The RMSNorm + projection launch given the producer's chunk sums gives
    the bits of the same launch summing the rows itself (one kernel at M <= 8;
    the activation prologue at M = 12, which ignores the sums)."""
    from nanopointllm_amd import _lib, w8a8

    hidden = 4096
    n = 12288 if proj == "qkv" else 22016
    epi = _lib.EPI_DEQUANT if proj == "qkv" else _lib.EPI_SILU_MUL
    wo, swo, _ = _weights(hidden, hidden, seed=31 + m)
    wp, swp, _ = _weights(n, hidden, seed=37 + m)
    g = torch.Generator().manual_seed(41 + m)
    ctx = torch.randn(m, hidden, generator=g).half().to(cuda)
    res = torch.randn(m, hidden, generator=g).half().to(cuda)
    nw = (torch.rand(hidden, generator=g) + 0.5).half().to(cuda)
    note(f"rmsnorm on sums m={m} {proj}")
    layout = _lib.ROWS_INTERLEAVE_HALVES if proj == "gateup" else _lib.ROWS_AS_IS
    summed = w8a8.linear_residual(ctx, w8a8.pack_rows(wo.to(cuda)), torch.from_numpy(swo).to(cuda),
                                  None, hidden, res)
    wpk = w8a8.pack_rows(wp.to(cuda), layout)
    swt = torch.from_numpy(swp).to(cuda)
    on_sums = w8a8.rmsnorm_linear(summed.y, nw, 1e-6, wpk, swt, None, n, epilogue=epi,
                                  ss_parts=summed.ss_parts)
    on_rows = w8a8.rmsnorm_linear(summed.y, nw, 1e-6, wpk, swt, None, n, epilogue=epi)
    assert torch.equal(on_sums.y, on_rows.y)
    # And the same as the residual add inside the norm launch (the route the
    # sums replace).
    o = w8a8.linear_dynamic(ctx, w8a8.pack_rows(wo.to(cuda)), torch.from_numpy(swo).to(cuda),
                            None, hidden)
    carried = w8a8.rmsnorm_linear(o, nw, 1e-6, wpk, swt, None, n, epilogue=epi, residual=res)
    assert torch.equal(carried.residual, summed.y)
    assert torch.equal(carried.y, on_sums.y)


def test_residual_stream_under_graph_capture(cuda):
    """The residual-add linear and the norm on its sums captured in a HIP
    graph: every replay equals the eager result."""
    from nanopointllm_amd import w8a8

    m, hidden, n = 8, 4096, 12288
    wo, swo, _ = _weights(hidden, hidden, seed=51)
    wp, swp, _ = _weights(n, hidden, seed=52)
    g = torch.Generator().manual_seed(53)
    ctx = torch.randn(m, hidden, generator=g).half().to(cuda)
    res = torch.randn(m, hidden, generator=g).half().to(cuda)
    nw = (torch.rand(hidden, generator=g) + 0.5).half().to(cuda)
    wop, swot = w8a8.pack_rows(wo.to(cuda)), torch.from_numpy(swo).to(cuda)
    wpk, swt = w8a8.pack_rows(wp.to(cuda)), torch.from_numpy(swp).to(cuda)

    def step():
        s = w8a8.linear_residual(ctx, wop, swot, None, hidden, res)
        return w8a8.rmsnorm_linear(s.y, nw, 1e-6, wpk, swt, None, n, ss_parts=s.ss_parts).y

    note("residual stream graph capture m=8")
    eager = step().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        step()  # eager work between replays
        torch.cuda.synchronize()
