"""The GEMV at 17..64 rows (csrc/gemv.hip), the regime of continuously
batched decode steps (engine/scheduler.py:46-100) through the projections of
paged_attention.py:97-124 and lightweight_runner.py:38-54, 329-379.

Two kernels serve it: with K <= 4096 and the int32 / dequant / SiLU*mul
epilogues the persistent gemv_rows_kernel (each wavefront keeps the x
fragments of its k-range in registers; one workgroup per CU, several blocks
each, or one block per CU at N = 4096, or fewer workgroups than CUs), and
otherwise gemv_kernel (three blocks per workgroup past 512 blocks).

Bars: int32 accumulators bit-exact against the oracle's integer product;
dequant outputs bit-equal to the oracle's binary32 result rounded once; the
SiLU*mul epilogue equal to the oracle's, its int8 twin equal to the oracle's
quantization of h, and its per-block row maxima giving the two-phase hq
bit-exact; requant1 and the single-rounding bf16 dequant exact.  Block counts
that leave a partial group (N = 12272 and 12290), K off the 64 grid, row
counts that leave a partial row tile (17, 33, 63) and fewer blocks than CUs
are included.
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


def _rows_kernel(m: int, n: int, k: int) -> bool:
    # gemv_rows_kernel's shapes (its int32 / dequant / SiLU*mul epilogues).
    return 16 < m <= 64 and k <= 4096


def _uses_gemv(m: int, n: int, k: int) -> bool:
    # The library's routing: the GEMV up to 32 rows, and up to 64 for
    # N <= 12288 or K <= 4096.
    return m <= 32 or (m <= 64 and (n <= 12288 or k <= 4096))


ROWS_SHAPES = [
    # (m, n, k) on gemv_rows_kernel: LLaMA-7B QKV at every row count of the
    # regime, a partial group of blocks (767 and 769 blocks), K off the 64
    # grid, one block per CU (N = 4096), fewer blocks than CUs, and the
    # widest N at 32 rows.
    (17, 12288, 4096), (24, 12288, 4096), (32, 12288, 4096), (33, 12288, 4096),
    (48, 12288, 4096), (64, 12288, 4096), (40, 12272, 1000), (32, 12290, 1000),
    (20, 9000, 130), (64, 8200, 72), (32, 4096, 4096), (64, 4096, 4000), (17, 1000, 64),
    (63, 300, 4096), (32, 22016, 4096), (48, 22016, 4096), (64, 22016, 4096),
]
OLD_SHAPES = [
    # gemv_kernel: K > 4096, three blocks per workgroup (MT = 2 and 4) and
    # one block per workgroup at 256 blocks.
    (24, 12288, 4160), (48, 12272, 5000), (40, 4096, 11008),
]


@pytest.mark.parametrize("m,n,k", ROWS_SHAPES + OLD_SHAPES)
def test_gemv_rows_int32_and_dequant(cuda, m, n, k):
    from nanopointllm_amd import w8a8

    assert _uses_gemv(m, n, k)
    xq, wq, sx, sw, bias = _case(m, n, k, seed=m + n + k)
    note(f"gemv rows m={m} n={n} k={k} rows_kernel={_rows_kernel(m, n, k)}")
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
                                      (48, 6000, 4096), (64, 4000, 2000), (29, 4500, 700),
                                      (48, 11008, 4096), (64, 11008, 4096),
                                      (33, 2000, 1000), (20, 11008, 4160)])
def test_gemv_rows_silu_mul_and_two_phase(cuda, m, inter, k):
    from nanopointllm_amd import _lib, w8a8

    n = 2 * inter
    assert _uses_gemv(m, n, k)
    xq, wq, sx, sw, _ = _case(m, n, k, seed=11 + k + m)
    note(f"gemv rows silu m={m} inter={inter} k={k} rows_kernel={_rows_kernel(m, n, k)}")
    wp = w8a8.pack_rows(wq.to(cuda), _lib.ROWS_INTERLEAVE_HALVES)
    sp = O.pack_gateup_rows(sw[:inter, None], sw[inter:, None], "interleave")[:, 0]
    qp = O.pack_gateup_rows(wq.numpy()[:inter], wq.numpy()[inter:], "interleave")
    xd, sxt = xq.to(cuda), torch.from_numpy(sx).to(cuda)
    spt = torch.from_numpy(np.ascontiguousarray(sp)).to(cuda)
    acc = O.int32_matmul_f64(xq.numpy(), qp)
    eh = O.gateup_silu_mul_from_acc(acc, sx, sp, layout="interleave")
    # bfloat16 chain: g and u rounded to bfloat16, then the reference's act_fn
    # (torch's CPU F.silu) and the product on bfloat16 tensors.
    yb = torch.from_numpy(O.dequant_epilogue(acc, sx, sp)).to(torch.bfloat16)
    ebh = (torch.nn.functional.silu(yb[:, 0::2]) * yb[:, 1::2]).float().numpy()
    hb = w8a8.linear_i8in(xd, sxt, wp, spt, None, n, epilogue=_lib.EPI_SILU_MUL,
                          out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(hb.float().cpu().numpy(), ebh)
    h = w8a8.linear_i8in(xd, sxt, wp, spt, None, n, epilogue=_lib.EPI_SILU_MUL,
                         out_dtype=torch.float16)
    np.testing.assert_array_equal(h.cpu().numpy(), eh.astype(np.float16))
    h_scale = float(O.static_activation_scale(float(h.float().abs().max().item())))
    hq = w8a8.linear_i8in(xd, sxt, wp, spt, None, n, epilogue=_lib.EPI_SILU_MUL_Q8,
                          out_dtype=torch.int8, y_scale=h_scale)
    eq = O.quantize_symmetric(h.cpu().numpy().astype(np.float32), np.float32(h_scale))
    np.testing.assert_array_equal(hq.cpu().numpy(), eq)
    out = w8a8.gateup_silu_mul_two_phase(xd, wp, spt, None, n, x_scale=sxt, in_features=k)
    np.testing.assert_array_equal(out.h.cpu().numpy(), h.cpu().numpy())
    tq, ts = O.dynamic_per_token_quant(h.cpu().numpy().astype(np.float32))
    np.testing.assert_array_equal(out.hq.cpu().numpy(), tq)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), ts[:, 0])


@pytest.mark.parametrize("m,n,k", [(24, 12290, 1000), (48, 12288, 4096)])
def test_gemv_rows_integer_epilogues(cuda, m, n, k):
    """requant1 and the single-rounding bf16 dequant stay on gemv_kernel at
    every K (gemv_rows_kernel does not take them)."""
    from nanopointllm_amd import _lib, integer_epilogues as E, w8a8

    xq, wq, sx, sw, _ = _case(m, n, k, seed=3 + m)
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


def test_gemv_rows_strided_and_padded_rows(cuda):
    """Caller int8 rows with a leading dimension past K (read in place when
    K % 64 == 0, else padded into the workspace) give the bits of contiguous
    rows."""
    from nanopointllm_amd import w8a8

    for m, n, k, ld in [(40, 12288, 4096, 4160), (33, 5000, 1000, 1040)]:
        xq, wq, sx, sw, bias = _case(m, n, k, seed=7 + m)
        note(f"gemv rows strided m={m} n={n} k={k} ld={ld}")
        big = torch.zeros((m, ld), dtype=torch.int8)
        big[:, :k] = xq
        xd = big.to(cuda)[:, :k]
        wp = w8a8.pack_rows(wq.to(cuda))
        sxt, swt, bt = (torch.from_numpy(a).to(cuda) for a in (sx, sw, bias))
        y = w8a8.linear_i8in(xd, sxt, wp, swt, bt, n, out_dtype=torch.float16)
        exp = O.dequant_epilogue(O.int32_matmul_f64(xq.numpy(), wq.numpy()), sx, sw, bias)
        np.testing.assert_array_equal(y.cpu().numpy(), exp.astype(np.float16))
