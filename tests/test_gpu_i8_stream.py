"""Decode GEMV on int8 activations with K > 8192: the fused kernel's
persistent weight stream, staging the given int8 rows instead of quantizing
(w8a8_linear_i8in / w8a8_linear / w8a8_gemm_i32 at M <= 8; the down
projection of lightweight_runner.py:362-379 and the int8 MLP chain).

Bars: int32 accumulators bit-exact against the oracle's integer product;
binary16 / bfloat16 / binary32 outputs bit-equal to the oracle's dequant
(w8a8.py:118-139) rounded once; SiLU*mul equal to the oracle's (torch's
``F.silu``, the reference's ``act_fn``); the int8 requant of SiLU*mul bit-exact against the oracle applied
to the kernel's own binary16 h.  Covered: K just above the threshold, K at its
maximum, K not a multiple of 64 (padded staging), strided rows, a partial last
output block, bias, every supported epilogue, and the K <= 8192 shapes that
stay on gemv_kernel.
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


def _case(m, n, k, seed, ldq=None):
    g = torch.Generator().manual_seed(seed)
    ldq = ldq or k
    xbuf = torch.randint(-127, 128, (m, ldq), generator=g, dtype=torch.int8)
    xq = xbuf[:, :k]
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    rng = np.random.default_rng(seed)
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((m, 1))) * 3).astype(np.float32)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return xbuf, xq, wq, sx, sw, bias


def _ulps16(a, b):
    def key(v):
        i = v.astype(np.float16).view(np.int16).astype(np.int32)
        return np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("m,n,k,ldq", [(1, 4100, 8256, None), (5, 4096, 11008, None),
                                       (8, 4100, 12288, None), (3, 2000, 12000, None),
                                       (8, 1600, 11008, 11072)])
def test_i8_stream_dequant_bias_and_int32(cuda, m, n, k, ldq):
    from nanopointllm_amd import w8a8

    xbuf, xq, wq, sx, sw, bias = _case(m, n, k, seed=m * 7 + k, ldq=ldq)
    note(f"i8 stream m={m} n={n} k={k} ldq={ldq}")
    xd = xbuf.to(cuda)[:, :k]
    wp = w8a8.pack_rows(wq.to(cuda))
    eacc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    acc = w8a8.gemm_i32(xd, wp, n)                       # int32 epilogue, no scales
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    sxt, swt, bt = (torch.from_numpy(a).to(cuda) for a in (sx, sw, bias))
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        for b in (None, bt):
            y = w8a8.linear_i8in(xd, sxt, wp, swt, b, n, out_dtype=dt)
            exp = O.dequant_epilogue(eacc, sx, sw, None if b is None else bias)
            got = y.float().cpu().numpy()
            if dt == torch.bfloat16:
                want = torch.from_numpy(exp).to(torch.bfloat16).float().numpy()
            else:
                want = exp.astype(np.float16).astype(np.float32) if dt == torch.float16 else exp
            np.testing.assert_array_equal(got, want, err_msg=f"{dt} bias={b is not None}")


@pytest.mark.parametrize("m", [1, 8])
def test_i8_stream_silu_and_int8_chain(cuda, m):
    from nanopointllm_amd import _lib, w8a8

    inter, k = 4104, 11008
    xbuf, xq, wq, sx, sw, _ = _case(m, 2 * inter, k, seed=40 + m)
    note(f"i8 stream silu m={m}")
    wp = w8a8.pack_rows(wq.to(cuda), _lib.ROWS_INTERLEAVE_HALVES)
    sp = O.pack_gateup_rows(sw[:inter, None], sw[inter:, None], "interleave")[:, 0]
    qp = O.pack_gateup_rows(wq.numpy()[:inter], wq.numpy()[inter:], "interleave")
    xd, sxt = xq.to(cuda), torch.from_numpy(sx).to(cuda)
    spt = torch.from_numpy(np.ascontiguousarray(sp)).to(cuda)
    h = w8a8.linear_i8in(xd, sxt, wp, spt, None, 2 * inter, epilogue=_lib.EPI_SILU_MUL,
                         out_dtype=torch.float16)
    eacc = O.int32_matmul_f64(xq.numpy(), qp)
    eh = O.gateup_silu_mul_from_acc(eacc, sx, sp, layout="interleave")
    u = _ulps16(h.cpu().numpy(), eh)
    assert u.max() == 0
    h_scale = float(O.static_activation_scale(float(h.float().abs().max().item())))
    hq = w8a8.linear_i8in(xd, sxt, wp, spt, None, 2 * inter, epilogue=_lib.EPI_SILU_MUL_Q8,
                          out_dtype=torch.int8, y_scale=h_scale)
    eq = O.quantize_symmetric(h.cpu().numpy().astype(np.float32), np.float32(h_scale))
    np.testing.assert_array_equal(hq.cpu().numpy(), eq)


def test_i8_stream_static_scale_broadcast_and_linear_path(cuda):
    """A per-tensor static scale (the int8 chain's h_scale) broadcast to every
    row, and w8a8_linear's quantize-then-GEMV route through the same stream."""
    from nanopointllm_amd import w8a8

    m, n, k = 8, 4096, 11008
    _, xq, wq, _, sw, _ = _case(m, n, k, seed=9)
    note("i8 stream static scale")
    wp, swt = w8a8.pack_rows(wq.to(cuda)), torch.from_numpy(sw).to(cuda)
    y = w8a8.linear_i8in(xq.to(cuda), torch.tensor([0.25], device=cuda), wp, swt, None, n)
    exp = O.dequant_epilogue(O.int32_matmul_f64(xq.numpy(), wq.numpy()),
                             np.full((m, 1), 0.25, np.float32), sw)
    np.testing.assert_array_equal(y.cpu().numpy(), exp.astype(np.float16))
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(3)) * 2).to(torch.float16)
    y = w8a8.linear_dynamic(x.to(cuda), wp, swt, None, n)
    eq, es = O.dynamic_per_token_quant(x.float().numpy())
    exp = O.dequant_epilogue(O.int32_matmul_f64(eq, wq.numpy()), es, sw)
    np.testing.assert_array_equal(y.cpu().numpy(), exp.astype(np.float16))


@pytest.mark.parametrize("k", [4096, 8192])
def test_short_k_stays_exact_on_gemv_kernel(cuda, k):
    from nanopointllm_amd import w8a8

    m, n = 8, 4096
    _, xq, wq, sx, sw, bias = _case(m, n, k, seed=k)
    note(f"i8 gemv k={k}")
    y = w8a8.linear_i8in(xq.to(cuda), torch.from_numpy(sx).to(cuda), w8a8.pack_rows(wq.to(cuda)),
                         torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda), n)
    exp = O.dequant_epilogue(O.int32_matmul_f64(xq.numpy(), wq.numpy()), sx, sw, bias)
    np.testing.assert_array_equal(y.cpu().numpy(), exp.astype(np.float16))
