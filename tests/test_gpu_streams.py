"""Launches on two streams at once share no state: the library keeps nothing
between calls but read-only device facts, so interleaved calls on two
default-priority streams (stream-ordered like the reference's call sites on
the current CUDA stream, engine/cuda_graph.py:30-46) give the bits that the
same calls give one after another.  Covered: the fused decode kernel (M = 8,
with and without the RMSNorm prologue), quantize + GEMV (M = 8, N = 4096),
and quantize + GEMM (M = 96, whose workspace is per call).
"""
from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _weights(cuda, n, k, seed):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(seed)
    wp = w8a8.pack_rows(torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(cuda))
    sw = (torch.rand(n, generator=g) * 0.01 + 1e-3).to(cuda)
    return wp, sw


def test_interleaved_streams_equal_sequential_calls(cuda):
    from nanopointllm_amd import w8a8

    k = 4096
    big = _weights(cuda, 12288, k, 1)     # fused decode kernel at M = 8
    small = _weights(cuda, 4096, k, 2)    # quantize + GEMV at M = 8, GEMM at M = 96
    nw = (1 + 0.1 * torch.randn(k, generator=torch.Generator().manual_seed(3))).half().to(cuda)
    g = torch.Generator().manual_seed(4)
    inputs = [(torch.randn(m, k, generator=g) * 2).half().to(cuda) for m in (8, 8, 96, 8, 96, 8)]

    def calls(x):
        """Three products on x: W8A8 linear, RMSNorm + linear, and on the
        small weight (a different route from the big one at M = 8)."""
        a = w8a8.linear_dynamic(x, big[0], big[1], None, 12288, in_features=k)
        b = w8a8.rmsnorm_linear(x, nw, 1e-6, big[0], big[1], None, 12288, in_features=k).y
        c = w8a8.linear_dynamic(x, small[0], small[1], None, 4096, in_features=k)
        return a, b, c

    note("sequential reference calls on the current stream")
    want = [calls(x) for x in inputs]
    torch.cuda.synchronize()

    note("the same calls interleaved on two streams, three rounds")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(3):
        got = [None] * len(inputs)
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for i, x in enumerate(inputs):
            with torch.cuda.stream(streams[i % 2]):
                got[i] = calls(x)
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for i, (w, o) in enumerate(zip(want, got)):
            for j, (u, v) in enumerate(zip(w, o)):
                assert torch.equal(u, v), f"input {i}, product {j}"
