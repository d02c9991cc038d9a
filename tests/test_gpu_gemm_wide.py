"""Prefill GEMM shapes past one round of 128x128 tiles, which select the
128-row tiles of 192, 224 or 256 columns (8 waves each, three LDS stages):
the widest whose tiles still fit in one round of workgroup slots, else (for
several rounds) 128x256, or from two full rounds of them the 256x256 tile
(16 waves, one workgroup per CU).

Bars as for every GEMM path: int32 accumulators bit-exact against the
oracle's integer product; binary16 / bfloat16 / binary32 dequant outputs
bit-equal to the oracle's dequant (w8a8.py:118-139) rounded once; SiLU*mul
equal to the oracle's (torch's ``F.silu``, the reference's ``act_fn``); the int8 requant of SiLU*mul
bit-exact against the oracle applied to the kernel's own binary16 h.  Shapes
are ragged in M, N and K (partial tiles, a partial last 16-row block, K not a
multiple of 64).  The integer requant epilogue (requant1) takes the same
tiles as the others.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from gemm_tiles import gemm_config
from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _ulps16(a, b):
    def key(v):
        i = v.astype(np.float16).view(np.int16).astype(np.int32)
        return np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(key(a) - key(b))


def _case(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    xq = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    rng = np.random.default_rng(seed)
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((m, 1))) * 3).astype(np.float32)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return xq, wq, sx, sw, bias


@pytest.mark.parametrize("m,n,k,cfg", [(1000, 14005, 200, "w224"), (2100, 6200, 320, "w224"),
                                        (1100, 20000, 576, "w256"), (1000, 12000, 330, "w192"),
                                        (2040, 16380, 200, "w256sq")])
def test_wide_tile_int32_and_dequant(cuda, m, n, k, cfg):
    from nanopointllm_amd import w8a8

    assert gemm_config(m, n) == cfg
    xq, wq, sx, sw, bias = _case(m, n, k, seed=m + n + k)
    note(f"gemm {cfg} m={m} n={n} k={k}")
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    eacc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    np.testing.assert_array_equal(w8a8.gemm_i32(xd, wp, n).cpu().numpy(), eacc)
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


@pytest.mark.parametrize("m,inter,k,cfg", [(1000, 7002, 320, "w224"), (1100, 10000, 200, "w256"),
                                            (1000, 6000, 330, "w192"), (2040, 8190, 136, "w256sq")])
def test_wide_tile_silu_mul_and_int8_chain(cuda, m, inter, k, cfg):
    from nanopointllm_amd import _lib, w8a8

    assert gemm_config(m, 2 * inter) == cfg
    xq, wq, sx, sw, _ = _case(m, 2 * inter, k, seed=11 + k)
    note(f"gemm {cfg} silu m={m} inter={inter} k={k}")
    wp = w8a8.pack_rows(wq.to(cuda), _lib.ROWS_INTERLEAVE_HALVES)
    sp = O.pack_gateup_rows(sw[:inter, None], sw[inter:, None], "interleave")[:, 0]
    qp = O.pack_gateup_rows(wq.numpy()[:inter], wq.numpy()[inter:], "interleave")
    xd, sxt = xq.to(cuda), torch.from_numpy(sx).to(cuda)
    spt = torch.from_numpy(np.ascontiguousarray(sp)).to(cuda)
    h = w8a8.linear_i8in(xd, sxt, wp, spt, None, 2 * inter, epilogue=_lib.EPI_SILU_MUL,
                         out_dtype=torch.float16)
    eh = O.gateup_silu_mul_from_acc(O.int32_matmul_f64(xq.numpy(), qp), sx, sp,
                                    layout="interleave")
    u = _ulps16(h.cpu().numpy(), eh)
    assert u.max() == 0
    h_scale = float(O.static_activation_scale(float(h.float().abs().max().item())))
    hq = w8a8.linear_i8in(xd, sxt, wp, spt, None, 2 * inter, epilogue=_lib.EPI_SILU_MUL_Q8,
                          out_dtype=torch.int8, y_scale=h_scale)
    eq = O.quantize_symmetric(h.cpu().numpy().astype(np.float32), np.float32(h_scale))
    np.testing.assert_array_equal(hq.cpu().numpy(), eq)


@pytest.mark.parametrize("m,n,k,cfg", [(1000, 14005, 200, "w224"), (1100, 20000, 200, "w256"),
                                        (2048, 16384, 264, "w256sq")])
def test_requant1_epilogue_at_a_wide_shape(cuda, m, n, k, cfg):
    """The integer requant epilogue on the wide tiles: equal to
    requantize_int32 of the exact product (that kernel is pinned to the
    oracle elsewhere), and a random sample of entries against the oracle."""
    from nanopointllm_amd import integer_epilogues as E, w8a8

    assert gemm_config(m, n) == cfg
    xq, wq, _, sw, _ = _case(m, n, k, seed=5)
    comp = [O.compile_fp16_requant_scale(0.02, float(w), 0.5) for w in sw]
    mult = np.array([c[0] for c in comp], np.uint32)
    shift = np.array([c[1] for c in comp], np.int32)
    bias = np.random.default_rng(5).integers(-3000, 3000, n).astype(np.int32)
    note(f"gemm {cfg} requant1 m={m} n={n} k={k}")
    multt = torch.from_numpy(mult.view(np.int32)).to(cuda)
    shiftt, biast = torch.from_numpy(shift).to(cuda), torch.from_numpy(bias).to(cuda)
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    y = E.linear_i8in_requant(xd, wp, multt, shiftt, biast, n).cpu().numpy()
    acc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    ref = E.requantize_int32(torch.from_numpy(acc).to(cuda), biast, multt, shiftt)
    np.testing.assert_array_equal(y, ref.cpu().numpy())
    rng = np.random.default_rng(6)
    for i, j in zip(rng.integers(0, m, 2000), rng.integers(0, n, 2000)):
        assert y[i, j] == O.requantize_int32(int(acc[i, j]), int(bias[j]), int(mult[j]),
                                             int(shift[j]))
