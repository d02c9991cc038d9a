"""w8a8_linear_noalloc (the entry point that allocates nothing) against
w8a8_linear with a caller workspace, through the C ABI.

Two calls in a row on the static scratch, the second with a smaller input
(so it runs over what the first left there), each bit-equal to w8a8_linear
on the same inputs; then the fused decode shape (no scratch at all), and a
problem larger than the scratch, which must be refused before any launch.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _case(m: int, n: int, k: int, seed: int, cuda):
    from nanopointllm_amd import w8a8
    import workloads as W

    x = W.prefill_activations(m, k, seed=seed, point_tokens=m // 2).to(cuda)
    g = torch.Generator().manual_seed(seed + 1)
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(cuda)
    sw = (torch.rand(n, generator=g) * 1e-3 + 1e-4).to(torch.float16).float().to(cuda)
    bias = torch.randn(n, generator=g).to(cuda)
    return x, w8a8.pack_rows(wq), sw, bias


def _call(fn_name: str, x, wp, sw, bias, n, epilogue, y, sx, workspace=None) -> int:
    from nanopointllm_amd import _lib

    lib = _lib.load()
    m, k = x.shape
    args = [x.data_ptr(), _lib.dtype_code(x.dtype), k, wp.data_ptr(), sw.data_ptr(),
            None if bias is None else bias.data_ptr(), epilogue, y.data_ptr(),
            _lib.dtype_code(y.dtype), y.shape[1], ctypes.c_float(0.0), _lib.F16, m, n, k,
            sx.data_ptr()]
    if fn_name == "w8a8_linear":
        args += [workspace.data_ptr(), workspace.numel()]
    return getattr(lib, fn_name)(*args, _lib.stream_handle(x.device))


def _both(m, n, k, seed, epilogue, out_dtype, cuda):
    from nanopointllm_amd import w8a8

    x, wp, sw, bias = _case(m, n, k, seed, cuda)
    b = bias if epilogue == 1 else None
    cols = n // 2 if epilogue in (2, 3) else n
    y_ref = torch.empty(m, cols, dtype=out_dtype, device=cuda)
    y = torch.full((m, cols), 7, dtype=out_dtype, device=cuda)
    sx_ref = torch.empty(m, dtype=torch.float32, device=cuda)
    sx = torch.empty(m, dtype=torch.float32, device=cuda)
    ws = torch.empty(w8a8.workspace_bytes(m, k), dtype=torch.uint8, device=cuda)
    note(f"noalloc vs linear m={m} n={n} k={k} epi={epilogue}")
    assert _call("w8a8_linear", x, wp, sw, b, n, epilogue, y_ref, sx_ref, ws) == 0
    assert _call("w8a8_linear_noalloc", x, wp, sw, b, n, epilogue, y, sx) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y_ref.cpu().numpy())
    np.testing.assert_array_equal(sx.cpu().numpy(), sx_ref.cpu().numpy())


def test_noalloc_matches_linear_on_two_calls(cuda):
    # GEMM regime (packed activations in the scratch), then a smaller GEMV
    # regime call (row-major activations over the first call's bytes).
    _both(560, 4096, 4096, 1, 1, torch.float16, cuda)
    _both(40, 1024, 1000, 2, 0, torch.int32, cuda)


def test_noalloc_fused_decode_and_silu(cuda):
    # Decode rows fused with the quantization (no scratch), and the SiLU*mul
    # epilogue on the GEMM regime.
    _both(8, 22016, 4096, 3, 2, torch.float16, cuda)
    _both(300, 2048, 512, 4, 2, torch.float16, cuda)


def test_noalloc_refuses_more_than_its_scratch(cuda):
    from nanopointllm_amd import _lib, w8a8

    m, k, n = 8192, 11008, 64
    assert w8a8.workspace_bytes(m, k) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(m, k, dtype=torch.float16, device=cuda)
    wp = torch.zeros(w8a8.packed_bytes(n, k), dtype=torch.int8, device=cuda)
    sw = torch.ones(n, device=cuda)
    y = torch.empty(m, n, dtype=torch.float16, device=cuda)
    sx = torch.empty(m, device=cuda)
    note("noalloc refuses an oversized problem")
    assert _call("w8a8_linear_noalloc", x, wp, sw, None, n, 1, y, sx) == _lib.ERR_TOO_LARGE


def test_noalloc_graph_replays_equal_eager(cuda):
    """Captured in a HIP graph (GEMM regime, so the scratch holds the packed
    activations) and replayed with eager work between replays: every replay
    equals the eager call bit for bit.  The eager call comes first, so the
    scratch address is resolved outside the capture."""
    m, n, k = 560, 4096, 4096
    x, wp, sw, bias = _case(m, n, k, 5, cuda)
    y_eager = torch.empty(m, n, dtype=torch.float16, device=cuda)
    sx_eager = torch.empty(m, dtype=torch.float32, device=cuda)
    note("noalloc graph capture m=560")
    assert _call("w8a8_linear_noalloc", x, wp, sw, bias, n, 1, y_eager, sx_eager) == 0
    torch.cuda.synchronize()
    y = torch.full((m, n), 3, dtype=torch.float16, device=cuda)
    sx = torch.empty(m, dtype=torch.float32, device=cuda)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert _call("w8a8_linear_noalloc", x, wp, sw, bias, n, 1, y, sx) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _call("w8a8_linear_noalloc", x, wp, sw, bias, n, 1, y, sx)
    assert rc == 0
    for rep in range(3):
        y.fill_(7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), rep
        assert torch.equal(sx, sx_eager), rep
        # Eager work on the same scratch between replays: a smaller GEMV-regime call.
        x2, wp2, sw2, _ = _case(40, 1024, 1000, 6 + rep, cuda)
        y2 = torch.empty(40, 1024, dtype=torch.int32, device=cuda)
        sx2 = torch.empty(40, dtype=torch.float32, device=cuda)
        assert _call("w8a8_linear_noalloc", x2, wp2, sw2, None, 1024, 0, y2, sx2) == 0
        torch.cuda.synchronize()
