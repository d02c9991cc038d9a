"""RMSNorm (and the residual add) in front of a W8A8 linear, one launch at
decode shapes: ``w8a8_rmsnorm_linear`` (LightweightRMSNorm,
lightweight_runner.py:239-257, then per-token dynamic quantization,
w8a8.py:106-115, and the per-output linear, w8a8.py:118-139; the W8A8 form of
``_rmsnorm_packed_qkv_kernel``, paged_attention.py:163-234).

Bars:
* at decode shapes (m <= 8, k <= 4096, enough weight per CU) the call needs
  no workspace: it is the one fused kernel;
* every route (the fused kernel; the prologue writing the GEMV's rows or the
  GEMM's packed tiles, then the product) gives the same bits as the
  activation prologue + the int8-in linear (outputs, summed residual,
  normalized rows, per-row scales), so a row's result does not depend on the
  batch it runs in;
* the residual add is bit-exact against the oracle; the normalized rows are
  bit-exact where the binary32 sum of squares is exact in any order, and on
  general inputs > 99.9 % bit-equal: torch's CPU ``mean`` sums in another
  order, which can move ``x / rms`` by one 16-bit ulp before the multiply by
  the norm weight; with weights in [0.5, 1.5) that is at most 2 ulps of the
  row;
* the quantization of the kernel's own rows is bit-exact, the int32
  accumulators exact, the dequant outputs bit-equal to the oracle's binary32
  result rounded once, and SiLU*mul equal to the oracle's (torch's ``F.silu``);
* graph replays equal the eager result, replay after replay.
"""
from __future__ import annotations

import ctypes
import functools
import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

TDT = {"f16": torch.float16, "bf16": torch.bfloat16}
HIDDEN, INTER = 4096, 11008


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _ulps(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(TDT[dtype]).view(torch.int16)
    u = torch.from_numpy(np.ascontiguousarray(b, np.float32)).to(TDT[dtype]).view(torch.int16)
    key = lambda i: torch.where(i < 0, -(i.int() & 0x7FFF), i.int())
    return (key(t) - key(u)).abs().numpy()


@functools.lru_cache(maxsize=6)
def _weights(proj: str, k: int = HIDDEN):
    """int8 [N, K] and binary32 scales [N] quantized per output row by the
    oracle (gate/up in the interleaved packed row order), and a bias."""
    import workloads as W

    if proj == "gateup":
        _, qg, sg = O.per_output_weight_qdq(W.linear_weight(INTER, k, seed=61).float().numpy())
        _, qu, su = O.per_output_weight_qdq(W.linear_weight(INTER, k, seed=62).float().numpy())
        q = O.pack_gateup_rows(qg, qu, "interleave")
        s = O.pack_gateup_rows(sg[:, None], su[:, None], "interleave")[:, 0]
    else:
        n = {"qkv": 3 * k, "small": 1024}[proj]
        _, q, s = O.per_output_weight_qdq(W.linear_weight(n, k, seed=n % 97).float().numpy())
    bias = (np.random.default_rng(q.shape[0]).standard_normal(q.shape[0]) * 0.1).astype(np.float32)
    return q, s, bias


def _device(proj: str, cuda, k: int = HIDDEN):
    from nanopointllm_amd import w8a8

    q, s, b = _weights(proj, k)
    return (w8a8.pack_rows(torch.from_numpy(q).to(cuda)), torch.from_numpy(s).to(cuda),
            torch.from_numpy(b).to(cuda))


def _rows(m: int, k: int, dtype: str, seed: int, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * scale
    x[:, : min(3, k)] *= 30          # outlier channels
    return x.to(TDT[dtype])


def _norm_weight(k: int, dtype: str, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(k, generator=g) + 0.5).to(TDT[dtype])


def _c_call(x, residual, norm_w, wp, sw, bias, n, epilogue, y, *, res_out=None, rows=None,
            sx_out=None, workspace=None, eps=1e-6) -> int:
    """One w8a8_rmsnorm_linear call through the C ABI; returns its status."""
    from nanopointllm_amd import _lib

    lib = _lib.load()
    m, k = x.shape
    ptr = lambda t: None if t is None else t.data_ptr()
    return lib.w8a8_rmsnorm_linear(
        x.data_ptr(), _lib.dtype_code(x.dtype), k, ptr(residual), k, ptr(res_out), k,
        norm_w.data_ptr(), ctypes.c_float(eps), wp.data_ptr(), sw.data_ptr(), ptr(bias),
        epilogue, y.data_ptr(), _lib.dtype_code(y.dtype), y.shape[1], ctypes.c_float(0.0),
        _lib.F16, m, n, k, ptr(sx_out), ptr(rows), k, ptr(workspace),
        0 if workspace is None else workspace.numel(), _lib.stream_handle(x.device))


def _two_launch(x, residual, norm_w, wp, sw, bias, n, epilogue, out_dtype, eps=1e-6):
    """The activation prologue then the int8-in linear (the route prefill rows
    take)."""
    from nanopointllm_amd import w8a8

    pro = w8a8.prologue_quant(x, norm_weight=norm_w, eps=eps, residual=residual,
                              return_rows=True)
    y = w8a8.linear_i8in(pro.q, pro.scale.reshape(-1), wp, sw, bias, n, epilogue=epilogue,
                         out_dtype=out_dtype, inter_dtype=torch.float16)
    return y, pro


CASES = [
    # (label, proj, m, dtype, residual, fused)
    ("qkv", "qkv", 1, "f16", False, True),
    ("qkv", "qkv", 3, "f16", False, True),
    ("qkv", "qkv", 8, "f16", False, True),
    ("qkv-bf16", "qkv", 8, "bf16", False, True),
    ("qkv-res", "qkv", 4, "f16", True, True),
    ("gateup-res", "gateup", 1, "f16", True, True),
    ("gateup-res", "gateup", 8, "f16", True, True),
    ("gateup-res-bf16", "gateup", 8, "bf16", True, True),
    ("qkv-12rows", "qkv", 12, "f16", True, False),
    ("qkv-16rows", "qkv", 16, "bf16", False, False),
    ("small-res", "small", 8, "f16", True, False),   # too little weight per CU
    # prefill rows: the prologue writes the GEMV's rows or the GEMM's tiles
    ("small-gemv-40", "small", 40, "f16", True, False),
    ("qkv-gemm-96", "qkv", 96, "f16", False, False),
    ("gateup-gemm-567", "gateup", 567, "bf16", True, False),
]


@pytest.mark.parametrize("label,proj,m,dtype,with_res,fused", CASES)
def test_rmsnorm_linear_against_two_launches_and_oracle(cuda, label, proj, m, dtype, with_res,
                                                        fused):
    from nanopointllm_amd import _lib

    k = 512 if proj == "small" else HIDDEN
    q, s, b = _weights(proj, k)
    wp, sw, bias = _device(proj, cuda, k)
    n = q.shape[0]
    silu = proj == "gateup"
    epi = _lib.EPI_SILU_MUL if silu else _lib.EPI_DEQUANT
    tdt = TDT[dtype]
    x = _rows(m, k, dtype, seed=m + k)
    x[:, 7] = -0.0   # a -0 element: its normalized value is -0 on every route
    x[:, 9] = -0.0
    x = x.to(cuda)
    res = None
    if with_res:
        res = _rows(m, k, dtype, seed=7 * m, scale=0.3)
        res[:, 9] = -0.0   # -0 + -0 = -0
        res = res.to(cuda)
    nw = _norm_weight(k, dtype, seed=m).to(cuda)
    cols = n // 2 if silu else n
    y = torch.empty(m, cols, dtype=torch.float16, device=cuda)
    rows = torch.empty(m, k, dtype=tdt, device=cuda)
    res_out = torch.empty(m, k, dtype=tdt, device=cuda) if with_res else None
    sx = torch.empty(m, dtype=torch.float32, device=cuda)
    note(f"rmsnorm_linear {label} m={m} n={n} k={k} {dtype} residual={with_res}")
    rc = _c_call(x, res, nw, wp, sw, bias, n, epi, y, res_out=res_out, rows=rows, sx_out=sx)
    if fused:
        assert rc == _lib.OK                  # no workspace: the one fused kernel
    else:
        assert rc == _lib.ERR_WORKSPACE
        ws = torch.empty(_lib.load().w8a8_workspace_bytes(m, k), dtype=torch.uint8, device=cuda)
        rc = _c_call(x, res, nw, wp, sw, bias, n, epi, y, res_out=res_out, rows=rows, sx_out=sx,
                     workspace=ws)
        assert rc == _lib.OK
    # the same bits as the activation prologue + int8 linear (zero signs too)
    y2, pro = _two_launch(x, res, nw, wp, sw, bias, n, epi, torch.float16)
    bits = lambda t: t.view(torch.int16)
    assert torch.equal(bits(y), bits(y2))
    assert torch.equal(bits(rows), bits(pro.rows))
    assert torch.equal(sx, pro.scale.reshape(-1))
    assert bool((bits(rows)[:, 9] == bits(torch.tensor(-0.0, dtype=tdt))).all())
    if with_res:
        assert torch.equal(bits(res_out), bits(pro.residual))
    # against the oracle
    xs = x.float().cpu().numpy()
    summed = xs
    if with_res:
        summed = O.residual_add(xs, res.float().cpu().numpy(), dtype)
        np.testing.assert_array_equal(res_out.float().cpu().numpy(), summed)
    ey = O.rmsnorm(summed, nw.float().cpu().numpy(), 1e-6, dtype)
    got_rows = rows.float().cpu().numpy()
    d = _ulps(got_rows, ey, dtype)
    note(f"  rows: exact {np.mean(d == 0):.6f}, max ulp {d.max()}")
    assert d.max() <= 2 and np.mean(d == 0) > 0.999
    xq, es = O.dynamic_per_token_quant(got_rows)
    np.testing.assert_array_equal(sx.cpu().numpy(), es[:, 0])
    acc = O.int32_matmul_f64(xq, q)
    if silu:
        eh = O.gateup_silu_mul_from_acc(acc, es, s, b, layout="interleave")
        u = _ulps(y.float().cpu().numpy(), eh.astype(np.float32), "f16")
        note(f"  h: exact {np.mean(u == 0):.6f}, max ulp {u.max()}")
        assert u.max() == 0
    else:
        np.testing.assert_array_equal(y.cpu().numpy(),
                                      O.dequant_epilogue(acc, es, s, b).astype(np.float16))


@pytest.mark.parametrize("m,dtype", [(1, "f16"), (8, "f16"), (8, "bf16")])
def test_residual_rmsnorm_gateup_int8_h_in_one_launch(cuda, m, dtype):
    """The static int8 MLP chain's gate/up (lightweight_runner.py:362-379 with
    a calibrated h scale): residual add + RMSNorm + quantization + packed
    gate/up + SiLU*mul + int8 requant of h, the one fused kernel at decode
    shapes (no workspace).  The same bits as the activation prologue + the
    int8-in linear; int8 h equal to quantize_symmetric (w8a8.py:33-43) of the
    oracle's SiLU*mul (binary16) from the kernel's own normalized rows."""
    from nanopointllm_amd import _lib, w8a8

    q, s, b = _weights("gateup")
    wp, sw, bias = _device("gateup", cuda)
    n, k, tdt = q.shape[0], HIDDEN, TDT[dtype]
    x = _rows(m, k, dtype, seed=500 + m).to(cuda)
    res = _rows(m, k, dtype, seed=600 + m, scale=0.3).to(cuda)
    nw = _norm_weight(k, dtype, seed=700 + m).to(cuda)
    h_scale = float(O.scale_from_absmax(np.float32(2.5)))
    hq = torch.empty(m, n // 2, dtype=torch.int8, device=cuda)
    rows = torch.empty(m, k, dtype=tdt, device=cuda)
    res_out = torch.empty(m, k, dtype=tdt, device=cuda)
    sx = torch.empty(m, dtype=torch.float32, device=cuda)
    lib = _lib.load()
    note(f"rmsnorm_linear gate/up SiLU*mul + int8 h, m={m} {dtype}")
    rc = lib.w8a8_rmsnorm_linear(
        x.data_ptr(), _lib.dtype_code(tdt), k, res.data_ptr(), k, res_out.data_ptr(), k,
        nw.data_ptr(), ctypes.c_float(1e-6), wp.data_ptr(), sw.data_ptr(), bias.data_ptr(),
        _lib.EPI_SILU_MUL_Q8, hq.data_ptr(), _lib.I8, n // 2, ctypes.c_float(h_scale),
        _lib.dtype_code(tdt), m, n, k, sx.data_ptr(), rows.data_ptr(), k, None, 0,
        _lib.stream_handle(cuda))
    assert rc == _lib.OK                      # no workspace: the one fused kernel
    pro = w8a8.prologue_quant(x, norm_weight=nw, eps=1e-6, residual=res, return_rows=True)
    hq2 = w8a8.linear_i8in(pro.q, pro.scale.reshape(-1), wp, sw, bias, n,
                           epilogue=_lib.EPI_SILU_MUL_Q8, out_dtype=torch.int8,
                           y_scale=h_scale, inter_dtype=tdt)
    bits = lambda t: t.view(torch.int16)
    assert torch.equal(hq, hq2)
    assert torch.equal(bits(rows), bits(pro.rows))
    assert torch.equal(bits(res_out), bits(pro.residual))
    assert torch.equal(sx, pro.scale.reshape(-1))
    if dtype == "f16":
        xq, es = O.dynamic_per_token_quant(rows.float().cpu().numpy())
        eh = O.gateup_silu_mul_from_acc(O.int32_matmul_f64(xq, q), es, s, b, layout="interleave")
        np.testing.assert_array_equal(hq.cpu().numpy(), O.quantize_symmetric(eh, h_scale))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("m", [1, 8])
def test_fused_accumulators_exact_where_the_sum_is_exact(cuda, dtype, m):
    """Rows of multiples of 1/8 in [-6, 6]: every binary32 partial sum of
    squares is exact, so the normalized rows, their quantization and the int32
    accumulators are bit-exact against the oracle end to end."""
    from nanopointllm_amd import _lib

    q, _, _ = _weights("qkv")
    wp, sw, _ = _device("qkv", cuda)
    n = q.shape[0]
    g = torch.Generator().manual_seed(31 + m)
    x = (torch.randint(-32, 33, (m, HIDDEN), generator=g).float() / 8).to(TDT[dtype])
    r = (torch.randint(-16, 17, (m, HIDDEN), generator=g).float() / 8).to(TDT[dtype])
    nw = _norm_weight(HIDDEN, dtype, seed=5)
    acc = torch.empty(m, n, dtype=torch.int32, device=cuda)
    res_out = torch.empty(m, HIDDEN, dtype=TDT[dtype], device=cuda)
    rows = torch.empty_like(res_out)
    note(f"rmsnorm_linear exact-sum {dtype} m={m}")
    assert _c_call(x.to(cuda), r.to(cuda), nw.to(cuda), wp, sw, None, n, _lib.EPI_I32, acc,
                   res_out=res_out, rows=rows) == _lib.OK
    summed = O.residual_add(x.float().numpy(), r.float().numpy(), dtype)
    np.testing.assert_array_equal(res_out.float().cpu().numpy(), summed)
    ey = O.rmsnorm(summed, nw.float().numpy(), 1e-6, dtype)
    np.testing.assert_array_equal(rows.float().cpu().numpy(), ey)
    xq, _ = O.dynamic_per_token_quant(ey)
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(xq, q))


def test_python_wrapper_and_modules(cuda):
    """``rmsnorm_linear`` and the module methods the runner uses give the
    fused kernel's bits; prefill rows take the two-launch route."""
    from nanopointllm_amd import linear, w8a8

    H, D = 32, 128
    g = torch.Generator().manual_seed(4)
    projs = [torch.nn.Linear(HIDDEN, H * D, bias=False) for _ in range(3)]
    for p in projs:
        p.weight.data = (torch.randn(p.weight.shape, generator=g) * 0.02).to(torch.float16)
        p.to(cuda)
    qkv = linear.W8A8PackedQKV(*projs, num_heads=H, num_kv_heads=H, head_dim=D)

    class _Norm(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(_norm_weight(HIDDEN, "f16", 8).to(cuda))
            self.variance_epsilon = 1e-5

    norm = _Norm()
    for m in (1, 8, 40):
        x = _rows(m, HIDDEN, "f16", seed=m).to(cuda)
        note(f"project_rmsnorm m={m}")
        q, k, v = qkv.project_rmsnorm(x, norm)
        pro = w8a8.prologue_quant(x, norm_weight=norm.weight, eps=1e-5, return_rows=True)
        q2, k2, v2 = qkv.project(pro.rows)
        assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    lin = qkv.linear.weight_q
    with pytest.raises(ValueError, match="one value per hidden channel"):
        w8a8.rmsnorm_linear(x, norm.weight[:-8], 1e-5, lin.packed, lin.scale, None,
                            lin.out_features)
    with pytest.raises(ValueError, match="residual must match"):
        w8a8.rmsnorm_linear(x, norm.weight, 1e-5, lin.packed, lin.scale, None,
                            lin.out_features, residual=x[:, :64])


def test_fused_rmsnorm_graph_replays(cuda):
    """Captured in a graph and replayed with eager work between replays:
    every replay equals the eager result."""
    from nanopointllm_amd import _lib, w8a8

    wp, sw, bias = _device("gateup", cuda)
    n = 2 * INTER
    x = _rows(8, HIDDEN, "f16", seed=9).to(cuda)
    r = _rows(8, HIDDEN, "f16", seed=10, scale=0.3).to(cuda)
    nw = _norm_weight(HIDDEN, "f16", seed=11).to(cuda)
    run = lambda: w8a8.rmsnorm_linear(x, nw, 1e-6, wp, sw, bias, n, residual=r,
                                      epilogue=_lib.EPI_SILU_MUL)
    eager = run()
    note("fused rmsnorm graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.y, eager.y) and torch.equal(out.residual, eager.residual), rep
        _ = (x.float() * 2).sum().item()   # eager work between replays


def test_in_place_residual_update_takes_the_prologue_route(cuda):
    """residual_out == residual (and x_out == x) at a shape the one-kernel
    route would take: the call asks for a workspace (the prologue route, which
    reads each row before writing it) and gives the non-aliased call's bits."""
    from nanopointllm_amd import _lib

    wp, sw, bias = _device("gateup", cuda)
    n, m = 2 * INTER, 8
    x = _rows(m, HIDDEN, "f16", seed=21).to(cuda)
    r = _rows(m, HIDDEN, "f16", seed=22, scale=0.3).to(cuda)
    nw = _norm_weight(HIDDEN, "f16", seed=23).to(cuda)
    y_ref = torch.empty(m, INTER, dtype=torch.float16, device=cuda)
    res_ref = torch.empty_like(x)
    rows_ref = torch.empty_like(x)
    note("rmsnorm_linear in place")
    assert _c_call(x, r, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y_ref, res_out=res_ref,
                   rows=rows_ref) == _lib.OK
    ws = torch.empty(_lib.load().w8a8_workspace_bytes(m, HIDDEN), dtype=torch.uint8,
                     device=cuda)
    r2, y2 = r.clone(), torch.empty_like(y_ref)
    assert _c_call(x, r2, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y2,
                   res_out=r2) == _lib.ERR_WORKSPACE
    assert _c_call(x, r2, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y2, res_out=r2,
                   workspace=ws) == _lib.OK
    assert torch.equal(y2, y_ref) and torch.equal(r2, res_ref)
    x3, y3 = x.clone(), torch.empty_like(y_ref)
    assert _c_call(x3, None, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y3,
                   rows=x3) == _lib.ERR_WORKSPACE
    assert _c_call(x3, None, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y3, rows=x3,
                   workspace=ws) == _lib.OK
    y4, rows4 = torch.empty_like(y_ref), torch.empty_like(x)
    assert _c_call(x, None, nw, wp, sw, bias, n, _lib.EPI_SILU_MUL, y4, rows=rows4) == _lib.OK
    assert torch.equal(y3, y4) and torch.equal(x3, rows4)
