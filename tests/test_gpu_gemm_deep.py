"""Prefill GEMM shapes with at most one round of tiles, which select ring
stages of several k-blocks: past 64 rows, 64x32 tiles (stages of four
k-blocks, two workgroups per CU) when they fill one round on at least half
the CUs; else one-wave 32x32 tiles with stages of four k-blocks (256 K) when
there is at most one 64x64 tile per CU, else the 64x64 tile with stages of
four k-blocks when its tiles fit in two per CU, else the 128x128 tile with
stages of two k-blocks (128 K) and one workgroup per CU.

Bars as for every GEMM path: int32 accumulators bit-exact against the
oracle's integer product; binary16 / bfloat16 dequant outputs bit-equal to the
oracle's dequant (w8a8.py:118-139) rounded once; SiLU*mul equal to the oracle's
(torch's ``F.silu``, the reference's ``act_fn``), its int8 requant bit-exact against the oracle
applied to the kernel's own binary16 h; the integer requant epilogue equal to
requantize_int32 of the exact product.  K is ragged against the stages: last
stages with fewer k-blocks than the others, a K that is not a multiple of 64,
and a K of one partial k-block.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from gemm_tiles import gemm_config as _config
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


# (m, n, k, config).  K-blocks of 64: 4197 -> 66, 1000 -> 16, 70 -> 2,
# 3100 -> 49 (a last 128-K stage of one k-block), 4250 -> 67 (a last 256-K
# stage of three), 11008 -> 172, and 70 (one 256-K stage of two).
SHAPES = [
    (760, 4096, 4197, "big-deep"),
    (800, 4100, 3100, "big-deep"),
    (800, 4096, 70, "big-deep"),
    (1000, 4096, 1000, "big-deep"),
    (700, 4100, 70, "big-deep"),
    (130, 12288, 3100, "big-deep"),
    (300, 6000, 11008, "small-deep"),
    (300, 6000, 4250, "small-deep"),
    (100, 1000, 4250, "tiny-deep"),
    (64, 12288, 4250, "tiny-deep"),
    (48, 9000, 70, "tiny-deep"),
    (65, 8000, 70, "mid"),
    (128, 4096, 11008, "mid"),
    (96, 4100, 4197, "mid"),
    (200, 2048, 3100, "mid"),
    (256, 4096, 4250, "mid"),
]


@pytest.mark.parametrize("m,n,k,cfg", SHAPES)
def test_deep_stage_int32_and_dequant(cuda, m, n, k, cfg):
    from nanopointllm_amd import _lib, w8a8

    assert _config(m, n) == cfg
    xq, wq, sx, sw, bias = _case(m, n, k, seed=m + n + k)
    note(f"gemm {cfg} m={m} n={n} k={k}")
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    eacc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    np.testing.assert_array_equal(w8a8.gemm_i32(xd, wp, n).cpu().numpy(), eacc)
    sxt, swt, bt = (torch.from_numpy(a).to(cuda) for a in (sx, sw, bias))
    for dt in (torch.float16, torch.bfloat16):
        for b in (None, bt):
            y = w8a8.linear_i8in(xd, sxt, wp, swt, b, n, out_dtype=dt)
            exp = O.dequant_epilogue(eacc, sx, sw, None if b is None else bias)
            want = torch.from_numpy(exp).to(dt).float().numpy()
            np.testing.assert_array_equal(y.float().cpu().numpy(), want,
                                          err_msg=f"{dt} bias={b is not None}")
    # The GEMM kernel alone on packed activations (below 65 rows the router
    # gives these shapes to the GEMV).
    xp = w8a8.pack_rows(xd)
    got = w8a8.linear_packed(xp, sxt, m, k, wp, swt, None, n, epilogue=_lib.EPI_I32,
                             out_dtype=torch.int32)
    np.testing.assert_array_equal(got.cpu().numpy(), eacc)
    got = w8a8.linear_packed(xp, sxt, m, k, wp, swt, bt, n, out_dtype=torch.float16)
    want = O.dequant_epilogue(eacc, sx, sw, bias).astype(np.float16)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("m,inter,k", [(760, 2048, 4197), (300, 3000, 4250), (100, 500, 4250),
                                      (96, 2048, 4197)])
def test_deep_stage_silu_mul_and_int8_chain(cuda, m, inter, k):
    from nanopointllm_amd import _lib, w8a8

    cfg = _config(m, 2 * inter)
    assert cfg in ("big-deep", "small-deep", "tiny-deep", "mid")
    xq, wq, sx, sw, _ = _case(m, 2 * inter, k, seed=7 + k)
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


@pytest.mark.parametrize("m,n,k", [(760, 4096, 4197), (300, 6000, 4250), (100, 1000, 4250),
                                   (128, 4096, 3100)])
def test_deep_stage_requant1_epilogue(cuda, m, n, k):
    from nanopointllm_amd import integer_epilogues as E, w8a8

    assert _config(m, n) in ("big-deep", "small-deep", "tiny-deep", "mid")
    xq, wq, _, sw, _ = _case(m, n, k, seed=5 + k)
    comp = [O.compile_fp16_requant_scale(0.02, float(w), 0.5) for w in sw]
    mult = np.array([c[0] for c in comp], np.uint32)
    shift = np.array([c[1] for c in comp], np.int32)
    bias = np.random.default_rng(5).integers(-3000, 3000, n).astype(np.int32)
    note(f"gemm deep requant1 m={m} n={n} k={k}")
    multt = torch.from_numpy(mult.view(np.int32)).to(cuda)
    shiftt, biast = torch.from_numpy(shift).to(cuda), torch.from_numpy(bias).to(cuda)
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    y = E.linear_i8in_requant(xd, wp, multt, shiftt, biast, n).cpu().numpy()
    acc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    ref = E.requantize_int32(torch.from_numpy(acc).to(cuda), biast, multt, shiftt)
    np.testing.assert_array_equal(y, ref.cpu().numpy())
    rng = np.random.default_rng(6)
    for i, j in zip(rng.integers(0, m, 1000), rng.integers(0, n, 1000)):
        assert y[i, j] == O.requantize_int32(int(acc[i, j]), int(bias[j]), int(mult[j]),
                                             int(shift[j]))
