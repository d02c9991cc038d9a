"""The GEMV at 17..64 rows (csrc/gemv.hip): past 16 rows a workgroup owns
three 16-output weight blocks and every activation fragment it loads serves
all three, the regime of continuously batched decode steps
(engine/scheduler.py:46-100) through the projections of
paged_attention.py:97-124 and lightweight_runner.py:38-54, 329-379.

Bars: int32 accumulators bit-exact against the oracle's integer product;
dequant outputs bit-equal to the oracle's binary32 result rounded once; the
SiLU*mul epilogue equal to the oracle's and its per-block row maxima giving
the two-phase hq bit-exact; requant1 and the single-rounding bf16 dequant
exact.  Block counts that leave a partial group of three (N = 12272 and
12290: 767 and 769 blocks) and K that is not a multiple of 64 are included.
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


def _case(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    xq = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    wq = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    rng = np.random.default_rng(seed)
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((m, 1))) * 3).astype(np.float32)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(n)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    return xq, wq, sx, sw, bias


def _uses_gemv(m: int, n: int) -> bool:
    # The library's routing: the GEMV up to 32 rows, and up to 64 for N <= 12288.
    return m <= 32 or (m <= 64 and n <= 12288)


SHAPES = [
    # (m, n, k): LLaMA-7B QKV at every row count of the regime, a partial
    # group of blocks (767 and 769 blocks), K off the 64 grid, and many blocks at 17 and 32 rows.
    (17, 12288, 4096), (24, 12288, 4096), (32, 12288, 4096), (48, 12288, 4096),
    (64, 12288, 4096), (40, 12272, 1000), (32, 12290, 1000), (20, 9000, 130), (32, 22016, 4096),
    (64, 8200, 72),
]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemv_rows_int32_and_dequant(cuda, m, n, k):
    from nanopointllm_amd import w8a8

    assert _uses_gemv(m, n) and -(-n // 16) > 512
    xq, wq, sx, sw, bias = _case(m, n, k, seed=m + n + k)
    note(f"gemv rows m={m} n={n} k={k}")
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


@pytest.mark.parametrize("m,inter,k", [(17, 11008, 4096), (24, 11008, 4096), (32, 11008, 4096),
                                      (29, 4500, 700)])
def test_gemv_rows_silu_mul_and_two_phase(cuda, m, inter, k):
    from nanopointllm_amd import _lib, w8a8

    n = 2 * inter
    assert _uses_gemv(m, n) and -(-n // 16) > 512
    xq, wq, sx, sw, _ = _case(m, n, k, seed=11 + k + m)
    note(f"gemv rows silu m={m} inter={inter} k={k}")
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
    out = w8a8.gateup_silu_mul_two_phase(xd, wp, spt, None, n, x_scale=sxt, in_features=k)
    np.testing.assert_array_equal(out.h.cpu().numpy(), h.cpu().numpy())
    tq, ts = O.dynamic_per_token_quant(h.cpu().numpy().astype(np.float32))
    np.testing.assert_array_equal(out.hq.cpu().numpy(), tq)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), ts[:, 0])


def test_gemv_rows_integer_epilogues(cuda):
    from nanopointllm_amd import _lib, integer_epilogues as E, w8a8

    m, n, k = 24, 12290, 1000
    xq, wq, sx, sw, _ = _case(m, n, k, seed=3)
    comp = [O.compile_fp16_requant_scale(0.02, float(w), 0.5) for w in sw]
    mult = np.array([c[0] for c in comp], np.uint32)
    shift = np.array([c[1] for c in comp], np.int32)
    bias = np.random.default_rng(3).integers(-3000, 3000, n).astype(np.int32)
    note(f"gemv rows integer epilogues m={m} n={n} k={k}")
    multt = torch.from_numpy(mult.view(np.int32)).to(cuda)
    shiftt, biast = torch.from_numpy(shift).to(cuda), torch.from_numpy(bias).to(cuda)
    xd, wp = xq.to(cuda), w8a8.pack_rows(wq.to(cuda))
    acc = O.int32_matmul_f64(xq.numpy(), wq.numpy())
    y = E.linear_i8in_requant(xd, wp, multt, shiftt, biast, n).cpu().numpy()
    ref = E.requantize_int32(torch.from_numpy(acc).to(cuda), biast, multt, shiftt)
    np.testing.assert_array_equal(y, ref.cpu().numpy())
    sxt, swt = torch.from_numpy(sx).to(cuda), torch.from_numpy(sw).to(cuda)
    yb = w8a8.linear_i8in(xd, sxt, wp, swt, None, n, epilogue=_lib.EPI_DEQUANT_BF16_EXACT,
                          out_dtype=torch.bfloat16)
    sa_bits = sx[:, 0].astype(np.float16).view(np.uint16)
    sw_bits = sw.astype(np.float16).view(np.uint16)
    rng = np.random.default_rng(4)
    for i, j in zip(rng.integers(0, m, 500), rng.integers(0, n, 500)):
        want = O.dequantize_int32_to_bf16(int(acc[i, j]), int(sa_bits[i]), int(sw_bits[j]))
        got = int(yb[i, j].view(torch.int16).item()) & 0xFFFF
        assert got == want, (i, j)
