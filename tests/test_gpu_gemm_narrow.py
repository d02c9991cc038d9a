"""The narrow GEMM tiles (csrc/gemm.hip ``gemm_kernel``): 112 x 96 (14
wavefronts of 16 x 48, a 3-stage ring of three k-blocks) and 128 x 96 (8
wavefronts of 32 x 48, a 2-stage ring of four k-blocks), taken when one round
of them fills the CUs, as for the O and down projections at M ~ 465..640
(paged_attention.py:1376, 1488; lightweight_runner.py:362-379).

Bars as for every GEMM path: int32 accumulators bit-exact against the
oracle's integer product; dequant outputs bit-equal to the oracle's binary32
result rounded once; SiLU*mul equal to the oracle's; the int8 requant of h
and the integer requant (requant1) bit-exact; the two-phase per-block maxima
giving hq and scales bit-exact against the per-token quantization of h.
Shapes are ragged in M, N and K, including K of one or a few k-blocks (fewer
than a ring stage) and K that leaves a partial last stage.
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


def _case(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    xq = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    rng = np.random.default_rng(seed)
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((m, 1))) * 3).astype(np.float32)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return xq, wq, sx, sw, bias


SHAPES = [
    # (m, n, k, tile): ragged rows / columns, K from one k-block to 11008
    (560, 4096, 4096, "t112x96"), (560, 4096, 11008, "t112x96"), (470, 3900, 1000, "t112x96"),
    (500, 4090, 64, "t112x96"), (545, 4000, 130, "t112x96"),
    (567, 4096, 4096, "t128x96"), (640, 4090, 11008, "t128x96"), (600, 4096, 130, "t128x96"),
    (620, 4096, 64, "t128x96"), (580, 3950, 1111, "t112x96"),
]


@pytest.mark.parametrize("m,n,k,cfg", SHAPES)
def test_narrow_int32_and_dequant(cuda, m, n, k, cfg):
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


@pytest.mark.parametrize("m,inter,k,cfg", [(560, 2048, 4096, "t112x96"), (500, 2000, 333, "t112x96"),
                                            (567, 2048, 1000, "t128x96"), (630, 2048, 640, "t128x96")])
def test_narrow_silu_mul_int8_chain_and_two_phase(cuda, m, inter, k, cfg):
    from nanopointllm_amd import _lib, w8a8

    n = 2 * inter
    assert gemm_config(m, n) == cfg
    xq, wq, sx, sw, _ = _case(m, n, k, seed=11 + k)
    note(f"gemm {cfg} silu m={m} inter={inter} k={k}")
    wp = w8a8.pack_rows(wq.to(cuda), _lib.ROWS_INTERLEAVE_HALVES)
    sp = O.pack_gateup_rows(sw[:inter, None], sw[inter:, None], "interleave")[:, 0]
    qp = O.pack_gateup_rows(wq.numpy()[:inter], wq.numpy()[inter:], "interleave")
    xd, sxt = xq.to(cuda), torch.from_numpy(sx).to(cuda)
    spt = torch.from_numpy(np.ascontiguousarray(sp)).to(cuda)
    h = w8a8.linear_i8in(xd, sxt, wp, spt, None, n, epilogue=_lib.EPI_SILU_MUL,
                         out_dtype=torch.float16)
    eh = O.gateup_silu_mul_from_acc(O.int32_matmul_f64(xq.numpy(), qp), sx, sp,
                                    layout="interleave")
    np.testing.assert_array_equal(h.cpu().numpy(), eh.astype(np.float16))
    h_scale = float(O.static_activation_scale(float(h.float().abs().max().item())))
    hq = w8a8.linear_i8in(xd, sxt, wp, spt, None, n, epilogue=_lib.EPI_SILU_MUL_Q8,
                          out_dtype=torch.int8, y_scale=h_scale)
    eq = O.quantize_symmetric(h.cpu().numpy().astype(np.float32), np.float32(h_scale))
    np.testing.assert_array_equal(hq.cpu().numpy(), eq)
    # Two-phase per-token requant: the epilogue's per-block maxima of h.
    out = w8a8.gateup_silu_mul_two_phase(xd, wp, spt, None, n, x_scale=sxt, in_features=k)
    np.testing.assert_array_equal(out.h.cpu().numpy(), h.cpu().numpy())
    tq, ts = O.dynamic_per_token_quant(h.cpu().numpy().astype(np.float32))
    np.testing.assert_array_equal(out.hq.cpu().numpy(), tq)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), ts[:, 0])


@pytest.mark.parametrize("m,n,k,cfg", [(560, 4096, 1000, "t112x96"), (600, 4096, 2000, "t128x96")])
def test_narrow_integer_epilogues(cuda, m, n, k, cfg):
    """requant1 (multiplier / shift int8 out) and the single-rounding
    int32 -> bf16 dequant on the narrow tiles."""
    from nanopointllm_amd import _lib, integer_epilogues as E, w8a8

    assert gemm_config(m, n) == cfg
    xq, wq, sx, sw, _ = _case(m, n, k, seed=5 + k)
    comp = [O.compile_fp16_requant_scale(0.02, float(w), 0.5) for w in sw]
    mult = np.array([c[0] for c in comp], np.uint32)
    shift = np.array([c[1] for c in comp], np.int32)
    bias = np.random.default_rng(5).integers(-3000, 3000, n).astype(np.int32)
    note(f"gemm {cfg} integer epilogues m={m} n={n} k={k}")
    multt = torch.from_numpy(mult.view(np.int32)).to(cuda)
    shiftt, biast = torch.from_numpy(shift).to(cuda), torch.from_numpy(bias).to(cuda)
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    acc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    y = E.linear_i8in_requant(xd, wp, multt, shiftt, biast, n).cpu().numpy()
    ref = E.requantize_int32(torch.from_numpy(acc).to(cuda), biast, multt, shiftt)
    np.testing.assert_array_equal(y, ref.cpu().numpy())
    rng = np.random.default_rng(6)
    for i, j in zip(rng.integers(0, m, 500), rng.integers(0, n, 500)):
        assert y[i, j] == O.requantize_int32(int(acc[i, j]), int(bias[j]), int(mult[j]),
                                             int(shift[j]))
    sxt, swt = torch.from_numpy(sx).to(cuda), torch.from_numpy(sw).to(cuda)
    yb = w8a8.linear_i8in(xd, sxt, wp, swt, None, n, epilogue=_lib.EPI_DEQUANT_BF16_EXACT,
                          out_dtype=torch.bfloat16)
    sa_bits = sx[:, 0].astype(np.float16).view(np.uint16)
    sw_bits = sw.astype(np.float16).view(np.uint16)
    for i, j in zip(rng.integers(0, m, 500), rng.integers(0, n, 500)):
        want = O.dequantize_int32_to_bf16(int(acc[i, j]), int(sa_bits[i]), int(sw_bits[j]))
        got = int(yb[i, j].view(torch.int16).item()) & 0xFFFF
        assert got == want, (i, j)

