"""GPU parity: libw8a8_gfx950.so against the CPU oracle on identical inputs.

Bars: int8 / int32 results bit-exact; binary16 / bfloat16 / binary32 outputs
bit-equal to the oracle's binary32 result rounded once; SiLU*mul outputs
equal to the oracle's, which applies the reference's ``act_fn`` (torch's CPU
``F.silu``) to the same binary16 gate and up, with
the downstream int32 of the int8 chain bit-exact against the oracle fed the
GPU's own int8 ``h``.
"""
from __future__ import annotations

import functools
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def note(msg: str) -> None:
    """Name the case on stderr before its GPU work (survives a crashed run)."""
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def f16_to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def rand_i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


@functools.lru_cache(maxsize=4)
def weight_q(n, k, seed):
    """Seeded weight [n, k] and its per-output int8 quantization (cached: the
    arrays are only read)."""
    import workloads as W

    w = W.linear_weight(n, k, seed=seed)
    _, q, s = O.per_output_weight_qdq(w.float().numpy())
    return w, q, s


# ------------------------------------------------------------ quantization
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 4096), (16, 4096), (7, 100), (3, 11008), (33, 4096), (5, 3), (3, 20000), (2, 2048)])
def test_quant_rows_bit_exact(cuda, dtype, shape):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(hash(shape) % 1000)
    x = torch.randn(*shape, generator=g) * 3
    x[0, : min(4, shape[1])] *= 50
    if shape[0] > 2:
        x[1] = 0.0                      # all-zero row -> scale 2**-14
        x[2] *= 1e-6                    # tiny row -> scale clamps to 2**-14
    x = x.to(dtype)
    note(f"quant_rows {dtype} {shape}")
    q, s = w8a8.quant_rows(x.to(cuda))
    xn = x.float().numpy()
    eq, es = O.dynamic_per_token_quant(xn)
    np.testing.assert_array_equal(s.cpu().numpy(), es[:, 0])
    np.testing.assert_array_equal(q.cpu().numpy(), eq)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_quant_exhaustive_16bit_inputs(cuda, dtype):
    """Every finite 16-bit value against the oracle's binary32 division, one
    scale per row: binary16 scales take the division-free path, the last
    scale (0.1, not binary16-representable) the dividing path."""
    from nanopointllm_amd import w8a8

    allv = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
    vals = allv[torch.isfinite(allv.float())]
    scales = [2.0 ** -14, 2.0 ** -24, 0.0124359130859375, 1.0 / 127, 0.33325, 1.0, 7.5,
              1000.0, 0.1]
    s32 = np.array([np.float32(np.float16(v)) for v in scales[:-1]] + [np.float32(0.1)],
                   np.float32)
    x = vals.reshape(1, -1).expand(len(scales), -1).contiguous()
    note(f"quant exhaustive {dtype} {tuple(x.shape)}")
    q = w8a8.quantize_symmetric(x.to(cuda), torch.from_numpy(s32).reshape(-1, 1).to(cuda))
    exp = O.quantize_symmetric(x.float().numpy(), s32[:, None])
    np.testing.assert_array_equal(q.cpu().numpy(), exp)


def test_quant_ties_round_to_even(cuda):
    from nanopointllm_amd import w8a8

    s = np.float32(np.float16(0.25))
    vals = (np.arange(-130, 130) + 0.5).astype(np.float32) * s   # exact half-integers
    x = torch.from_numpy(vals.astype(np.float16)).reshape(1, -1)
    note("quant_rows_scaled ties")
    q = w8a8.quantize_symmetric(x.to(cuda), torch.tensor(float(s), device=cuda))
    np.testing.assert_array_equal(q.cpu().numpy(), O.quantize_symmetric(x.float().numpy(), s))


def test_quantize_symmetric_reference_kat(cuda):
    from nanopointllm_amd import w8a8

    kat = GOLDEN["rounding_clipping"]
    note("quantize_symmetric KAT")
    q = w8a8.quantize_symmetric(torch.tensor(kat["values"], device=cuda),
                                torch.tensor(kat["scale"], device=cuda))
    assert q.dtype == torch.int8
    assert q.cpu().tolist() == kat["asserted"]
    with pytest.raises(ValueError, match="positive"):
        w8a8.quantize_symmetric(torch.ones(1, device=cuda), torch.tensor(0.0, device=cuda))


def test_quantize_per_row_scales(cuda):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 257, generator=g).to(torch.float16)
    scales = torch.tensor(O.scale_from_absmax(np.abs(x.float().numpy()).max(1, keepdims=True)))
    note("quantize_symmetric per-row")
    q = w8a8.quantize_symmetric(x.to(cuda), scales.to(cuda))
    np.testing.assert_array_equal(q.cpu().numpy(),
                                  O.quantize_symmetric(x.float().numpy(), scales.numpy()))


def test_per_output_weight_qdq(cuda):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(4)
    w = torch.randn(5, 259, generator=g)
    note("per_output_weight_qdq")
    deq, q, s = w8a8.per_output_weight_qdq(w.to(cuda))
    edeq, eq, es = O.per_output_weight_qdq(w.numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(deq.cpu().numpy(), edeq)


# ------------------------------------------------------------------ packing
def _pack_numpy(q: np.ndarray, interleave: bool = False) -> np.ndarray:
    rows, k = q.shape
    src = q
    if interleave:
        half = rows // 2
        src = np.stack([q[:half], q[half:]], 1).reshape(rows, k)
    rp, kp = -(-rows // 16) * 16, -(-k // 64) * 64
    pad = np.zeros((rp, kp), np.int8)
    pad[:rows, :k] = src
    # [rb, r, kb, g, b] -> tile (rb, kb), lane r + 16 g, byte b
    t = pad.reshape(rp // 16, 16, kp // 64, 4, 16).transpose(0, 2, 3, 1, 4)
    return t.reshape(-1)


@pytest.mark.parametrize("rows,k", [(16, 64), (37, 200), (1, 4096), (48, 100)])
def test_pack_rows_layout(cuda, rows, k):
    from nanopointllm_amd import _lib, w8a8

    q = rand_i8((rows, k), rows * 7 + k)
    note(f"pack_rows {rows}x{k}")
    got = w8a8.pack_rows(q.to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(got, _pack_numpy(q.numpy()))
    if rows % 2 == 0:
        got = w8a8.pack_rows(q.to(cuda), _lib.ROWS_INTERLEAVE_HALVES).cpu().numpy()
        np.testing.assert_array_equal(got, _pack_numpy(q.numpy(), interleave=True))


# ----------------------------------------------------------- int32 products
GEMM_MS = [1, 2, 3, 8, 15, 16, 17, 31, 33, 64, 65, 100, 128, 129, 300]
GEMM_NK = [(48, 64), (50, 100), (16, 4096), (136, 320)]


@pytest.mark.parametrize("n,k", GEMM_NK)
@pytest.mark.parametrize("m", GEMM_MS)
def test_gemm_i32_exact(cuda, m, n, k):
    from nanopointllm_amd import w8a8

    a = rand_i8((m, k), m * 131 + n)
    w = rand_i8((n, k), n * 17 + k)
    note(f"gemm_i32 m={m} n={n} k={k}")
    acc = w8a8.gemm_i32(a.to(cuda), w8a8.pack_rows(w.to(cuda)), n)
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(a.numpy(), w.numpy()))


@pytest.mark.parametrize("m,n,k", [(300, 11000, 200), (129, 16400, 4096), (1000, 2050, 576)])
def test_gemm_large_tile_config_ragged(cuda, m, n, k):
    """Shapes that select the 128x128 / 16-wave GEMM tile with ragged M, N, K."""
    from nanopointllm_amd import w8a8

    a = rand_i8((m, k), m + 5)
    w = rand_i8((n, k), n + 7)
    note(f"gemm large tile m={m} n={n} k={k}")
    acc = w8a8.gemm_i32(a.to(cuda), w8a8.pack_rows(w.to(cuda)), n)
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(a.numpy(), w.numpy()))


def test_gemm_i32_extreme_values(cuda):
    from nanopointllm_amd import w8a8

    k = 11008
    a = torch.full((3, k), 127, dtype=torch.int8)
    a[1] = -127
    a[2, ::2] = -127
    w = torch.full((20, k), -127, dtype=torch.int8)
    w[5] = 127
    note("gemm_i32 extremes")
    acc = w8a8.gemm_i32(a.to(cuda), w8a8.pack_rows(w.to(cuda)), 20)
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(a.numpy(), w.numpy()))


def test_gemm_i32_unaligned_and_strided_input(cuda):
    from nanopointllm_amd import w8a8

    big = rand_i8((80, 130), 77)
    a = big[:, 1:101]            # leading dimension 130, odd byte offset
    w = rand_i8((30, 100), 78)
    wp = w8a8.pack_rows(w.to(cuda))
    big_d = big.to(cuda)
    for m in (8, 70):
        note(f"gemm_i32 strided m={m}")
        acc = w8a8.gemm_i32(big_d[:m, 1:101], wp, 30)
        np.testing.assert_array_equal(acc.cpu().numpy(),
                                      O.int32_matmul_f64(a[:m].numpy(), w.numpy()))


def test_package_fixture_on_gpu(cuda, tmp_path):
    from nanopointllm_amd import package

    pkg = GOLDEN["package"]
    package.write_quantized_linear_package(
        tmp_path, activation=np.array(pkg["activation"], np.int8),
        weight=np.array(pkg["weight"], np.int8),
        activation_scale=np.array([pkg["activation_scale"]], np.float16),
        weight_scale=np.array(pkg["weight_scale"], np.float16),
        smooth_scale=np.array(pkg["smooth_scale"], np.float16),
        output_scale=np.array([pkg["output_scale"]], np.float16), provenance=pkg["provenance"])
    loaded = package.load_quantized_linear_package(tmp_path)
    note("package golden on GPU")
    got = package.package_integer_golden_gpu(loaded, device=cuda).cpu().numpy()
    np.testing.assert_array_equal(got, np.array(pkg["derived_integer_golden"], np.int32))
    np.testing.assert_array_equal(got, loaded.integer_golden())


# --------------------------------------------------------------- linears
def _expected_linear(x: torch.Tensor, q: np.ndarray, s: np.ndarray, bias=None):
    out, acc, _, _ = O.w8a8_linear_dynamic(x.float().numpy(), q, s, bias)
    return out, acc


def test_config1_single_linear_bit_exact(cuda):
    """X fp16 [16,4096] with 8 outlier channels x20, W [4096,4096] ~N(0,0.02), seed 0."""
    from nanopointllm_amd import linear
    import workloads as W

    x, w = W.config1(seed=0)
    note("config1 M=16 4096x4096")
    lin = linear.W8A8Linear(linear.PackedW8A8Weight.from_float(w.to(cuda)))
    y = lin(x.to(cuda))
    acc = lin.accumulators(x.to(cuda))
    _, qw, sw = O.per_output_weight_qdq(w.float().numpy())
    exp, eacc = _expected_linear(x, qw, sw)
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))
    err = O.tensor_error(exp, f16_to_np(y).astype(np.float32))
    note(f"config1 fp16 vs oracle f32: {err}")


@pytest.mark.parametrize("m", [1, 4, 8, 16, 17, 40, 64, 65, 130, 560])
@pytest.mark.parametrize("n,k", [(64, 128), (48, 100), (200, 4096)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_fp16_bit_exact(cuda, m, n, k, with_bias):
    from nanopointllm_amd import w8a8

    x = torch.from_numpy(np.asarray(
        torch.randn(m, k, generator=torch.Generator().manual_seed(m + n)).numpy() * 2)).to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + k)
    bias = (np.linspace(-1, 1, n).astype(np.float32) if with_bias else None)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    note(f"linear fp16 m={m} n={n} k={k} bias={with_bias}")
    y = w8a8.linear_dynamic(x.to(cuda), wp, torch.from_numpy(sw).to(cuda),
                            None if bias is None else torch.from_numpy(bias).to(cuda), n)
    exp, _ = _expected_linear(x, qw, sw, bias)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


def _linear_without_workspace(x, wp, sw, bias, n, epi, y_dtype):
    """w8a8_linear with a null workspace: succeeds only on the fused decode
    kernel (every other path reports ERR_WORKSPACE before launching)."""
    from nanopointllm_amd import _lib

    lib = _lib.load()
    m, k = x.shape
    ncols = n // 2 if epi in (_lib.EPI_SILU_MUL, _lib.EPI_SILU_MUL_Q8) else n
    y = torch.empty(m, ncols, dtype=y_dtype, device=x.device)
    sx = torch.full((m,), -1.0, device=x.device)
    rc = lib.w8a8_linear(x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), wp.data_ptr(),
                         sw.data_ptr(), None if bias is None else bias.data_ptr(), epi,
                         y.data_ptr(), _lib.dtype_code(y_dtype), y.stride(0), 0.0, _lib.F16,
                         m, n, k, sx.data_ptr(), None, 0, _lib.stream_handle(x.device))
    return rc, y, sx


# Shapes the fused kernel takes on a 256-CU MI355X (per CU >= 64 KiB of
# weights and >= 4 weight bytes per quantized activation element): 3, 8, 32
# and 2 blocks per CU; K = 256 leaves 12 of the 16 wavefronts without a
# k-range, K = 12288 is the largest K the kernel takes.
@pytest.mark.parametrize("m", [1, 2, 3, 5, 7, 8])
@pytest.mark.parametrize("n,k", [(12288, 4096), (32768, 1000), (131072, 256), (8192, 12288)])
def test_fused_decode_path(cuda, m, n, k):
    """Workspace-free decode kernel (quantization fused in): outputs, row
    scales and int32 accumulators against the oracle."""
    from nanopointllm_amd import _lib, w8a8

    g = torch.Generator().manual_seed(m * 1000 + k)
    x = (torch.randn(m, k, generator=g) * 2.5)
    x[:, :: max(1, k // 7)] *= 30
    x = x.to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + 3)
    bias = np.linspace(-2, 2, n).astype(np.float32)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt, bt, xc = torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda), x.to(cuda)
    note(f"fused decode m={m} n={n} k={k}")
    rc, y, sx = _linear_without_workspace(xc, wp, swt, bt, n, _lib.EPI_DEQUANT, torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    rc, acc, _ = _linear_without_workspace(xc, wp, swt, None, n, _lib.EPI_I32, torch.int32)
    assert rc == 0
    exp, eacc, _, esx = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw, bias)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


@pytest.mark.parametrize("m", [9, 12, 13, 16])
@pytest.mark.parametrize("n,k", [(32768, 1000), (131072, 256), (24576, 4096), (20480, 6144),
                                 (12288, 4096)])
def test_fused_decode_16_rows(cuda, m, n, k):
    """9 to 16 rows on the workspace-free kernel (full 16-row A fragments,
    K <= 6144): outputs, row scales and int32 accumulators against the
    oracle."""
    from nanopointllm_amd import _lib, w8a8

    g = torch.Generator().manual_seed(m * 77 + k)
    x = (torch.randn(m, k, generator=g) * 2.0)
    x[:, :: max(1, k // 5)] *= 25
    x = x.to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + 11)
    bias = np.linspace(-1, 1, n).astype(np.float32)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt, bt, xc = torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda), x.to(cuda)
    note(f"fused decode 16 rows m={m} n={n} k={k}")
    rc, y, sx = _linear_without_workspace(xc, wp, swt, bt, n, _lib.EPI_DEQUANT, torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    rc, acc, _ = _linear_without_workspace(xc, wp, swt, None, n, _lib.EPI_I32, torch.int32)
    assert rc == 0
    exp, eacc, _, esx = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw, bias)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


@pytest.mark.parametrize("m", [10, 16])
def test_fused_decode_16_rows_silu_bf16_ties(cuda, m):
    """The SiLU*mul epilogue, bfloat16 x and integer activations whose every
    chunk holds exact ties, on the 16-row fused kernel."""
    from nanopointllm_amd import _lib, w8a8

    inter, k = 12288, 4096
    g = torch.Generator().manual_seed(m)
    x = (torch.randn(m, k, generator=g) * 3).to(torch.float16)
    _, qw, sw = weight_q(2 * inter, k, seed=m + 100)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda), _lib.ROWS_INTERLEAVE_HALVES)
    sp = O.pack_gateup_rows(sw[:inter, None], sw[inter:, None], "interleave")[:, 0]
    qp = O.pack_gateup_rows(qw[:inter], qw[inter:], "interleave")
    spt = torch.from_numpy(np.ascontiguousarray(sp)).to(cuda)
    note(f"fused decode 16 rows silu m={m}")
    rc, h, sx = _linear_without_workspace(x.to(cuda), wp, spt, None, 2 * inter, _lib.EPI_SILU_MUL,
                                          torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    eq, es = O.dynamic_per_token_quant(x.float().numpy())
    np.testing.assert_array_equal(sx.cpu().numpy(), es[:, 0])
    eh = O.gateup_silu_mul_from_acc(O.int32_matmul_f64(eq, qp), es, sp, layout="interleave")
    key = lambda v: (lambda i: np.where(i < 0, -(i & 0x7FFF), i))(
        v.astype(np.float16).view(np.int16).astype(np.int32))
    u = np.abs(key(f16_to_np(h)) - key(eh))
    assert u.max() == 0
    # bfloat16 x, dequant to bfloat16
    n = 2 * inter  # 6 blocks per CU: the routing takes the fused kernel up to M = 16
    wq = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swq = torch.from_numpy(sw).to(cuda)
    xb = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16)
    rc, yb, sxb = _linear_without_workspace(xb.to(cuda), wq, swq, None, n, _lib.EPI_DEQUANT,
                                            torch.bfloat16)
    assert rc == 0
    exp, _, _, esx = O.w8a8_linear_dynamic(xb.float().numpy(), qw, sw)
    np.testing.assert_array_equal(sxb.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(yb.float().cpu().numpy(),
                                  torch.from_numpy(exp).to(torch.bfloat16).float().numpy())
    # ties: integer activations with |x|max = 254 give s = 2
    xt = torch.randint(-254, 255, (m, k), generator=g).to(torch.float16)
    xt[:, 0] = 254
    rc, acc, sxt = _linear_without_workspace(xt.to(cuda), wq, swq, None, n, _lib.EPI_I32,
                                             torch.int32)
    assert rc == 0
    tq, ts = O.dynamic_per_token_quant(xt.float().numpy())
    np.testing.assert_array_equal(sxt.cpu().numpy(), ts[:, 0])
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(tq, qw))


@pytest.mark.parametrize("m", [1, 2, 4])
def test_fused_decode_o_shape_small_m(cuda, m):
    """The O projection (4096 x 4096, one 64 KiB block per CU) takes the
    workspace-free kernel at M <= 4: outputs, scales and accumulators."""
    from nanopointllm_amd import _lib, w8a8

    n, k = 4096, 4096
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(m)) * 3).to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=5)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt, xc = torch.from_numpy(sw).to(cuda), x.to(cuda)
    note(f"fused decode o-shape m={m}")
    rc, y, sx = _linear_without_workspace(xc, wp, swt, None, n, _lib.EPI_DEQUANT, torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    rc, acc, _ = _linear_without_workspace(xc, wp, swt, None, n, _lib.EPI_I32, torch.int32)
    assert rc == 0
    exp, eacc, _, esx = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


@pytest.mark.parametrize("m", [1, 3, 8])
def test_fused_decode_exact_ties(cuda, m):
    """Integer activations with |x|max = 254 give s = 2, so half the values
    are exact ties x/s = n + 1/2: the fused kernel's quantizer takes its exact
    fallback on almost every chunk and must still round ties to even."""
    from nanopointllm_amd import _lib, w8a8

    n, k = 12288, 4096
    g = torch.Generator().manual_seed(m)
    x = torch.randint(-254, 255, (m, k), generator=g).float()
    x[:, 0] = 254.0
    x = x.to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + 3)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt = torch.from_numpy(sw).to(cuda)
    note(f"fused decode ties m={m}")
    rc, acc, sx = _linear_without_workspace(x.to(cuda), wp, swt, None, n, _lib.EPI_I32,
                                            torch.int32)
    assert rc == 0
    xq, esx = O.dynamic_per_token_quant(x.float().numpy())
    assert float(esx[0, 0]) == 2.0
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(xq, qw))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 11008), (16, 11264), (1000, 4104),
                                 (4095, 5000), (40, 64), (16, 8)])
def test_split_decode_path(cuda, m, n, k):
    """At most one 16-output block per CU (N <= 16 * CUs), M <= 8, K <= 11264,
    the dequant epilogue: the workspace-free kernel whose wavefronts split
    into row quantizers and weight loaders (o_proj and down at decode).
    Outputs with a bias, row scales, and the binary32 output, against the
    oracle; K = 4104 and 5000 are the first k-blocks past the short-row
    variant, 11264 the largest K it takes, N = 16 one block."""
    from nanopointllm_amd import _lib, w8a8

    g = torch.Generator().manual_seed(m * 100 + k)
    x = torch.randn(m, k, generator=g) * 2.5
    x[:, :: max(1, k // 5)] *= 40
    x = x.to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + k)
    bias = np.linspace(-2, 2, n).astype(np.float32)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt, bt, xc = torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda), x.to(cuda)
    note(f"split decode m={m} n={n} k={k}")
    rc, y, sx = _linear_without_workspace(xc, wp, swt, bt, n, _lib.EPI_DEQUANT, torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    exp, _, _, esx = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw, bias)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))
    rc, y32, _ = _linear_without_workspace(xc, wp, swt, bt, n, _lib.EPI_DEQUANT, torch.float32)
    assert rc == 0
    np.testing.assert_array_equal(y32.cpu().numpy(), exp)


@pytest.mark.parametrize("m", [9, 10, 12, 13, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1000, 4096), (40, 64), (4095, 2000)])
def test_split_decode_path_16_rows(cuda, m, n, k):
    """9-16 rows of K <= 4096 on the split kernel (each row wavefront takes
    rows w and w + 8): outputs with a bias and row scales against the
    oracle, through the workspace-free call."""
    from nanopointllm_amd import _lib, w8a8

    g = torch.Generator().manual_seed(m * 31 + k)
    x = torch.randn(m, k, generator=g) * 2
    x[:, :: max(1, k // 3)] *= 25
    x = x.to(torch.float16)
    _, qw, sw = weight_q(n, k, seed=n + 2 * k)
    bias = np.linspace(-1, 1, n).astype(np.float32)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt, bt, xc = torch.from_numpy(sw).to(cuda), torch.from_numpy(bias).to(cuda), x.to(cuda)
    note(f"split decode 16 rows m={m} n={n} k={k}")
    rc, y, sx = _linear_without_workspace(xc, wp, swt, bt, n, _lib.EPI_DEQUANT, torch.float16)
    assert rc == 0, _lib.load().w8a8_status_string(rc)
    exp, _, _, esx = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw, bias)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx[:, 0])
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


@pytest.mark.parametrize("m,n,k", [(8, 4096, 4096), (3, 4096, 11008), (6, 700, 2000),
                                   (14, 4096, 4096)])
def test_split_decode_path_bf16(cuda, m, n, k):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(m + k)
    x = (torch.randn(m, k, generator=g) * 3).to(torch.bfloat16)
    _, qw, sw = weight_q(n, k, seed=k)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    note(f"split decode bf16 m={m} n={n} k={k}")
    y = w8a8.linear_dynamic(x.to(cuda), wp, torch.from_numpy(sw).to(cuda), None, n)
    exp, _, _, _ = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw)
    assert y.dtype == torch.bfloat16
    assert torch.equal(y.cpu(), torch.from_numpy(exp).to(torch.bfloat16))


def test_fused_path_not_taken_for_small_shapes(cuda):
    """Projections that neither fused kernel takes on a 256-CU MI355X (12
    rows of K = 4104 and 17 rows of K = 4096, beyond the split kernel's 16
    rows of K <= 4096; K = 12288 beyond its 8 rows; 257 blocks of short
    rows) and the int32 epilogue of the split shapes go through quantization
    + GEMV (they need a workspace) and give the same results."""
    from nanopointllm_amd import _lib, w8a8

    for m, n, k in [(12, 4096, 4104), (17, 4096, 4096), (8, 4096, 12288), (8, 4112, 1024)]:
        _, qw, sw = weight_q(n, k, seed=n + k)
        wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.float16)
        note(f"unfused decode m={m} n={n} k={k}")
        rc, _, _ = _linear_without_workspace(x.to(cuda), wp, torch.from_numpy(sw).to(cuda), None,
                                             n, _lib.EPI_DEQUANT, torch.float16)
        assert rc == _lib.ERR_WORKSPACE
        y = w8a8.linear_dynamic(x.to(cuda), wp, torch.from_numpy(sw).to(cuda), None, n)
        exp, _, _, _ = O.w8a8_linear_dynamic(x.float().numpy(), qw, sw)
        np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))
    m, n, k = 8, 4096, 4096
    _, qw, sw = weight_q(n, k, seed=n + k)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.float16)
    note("unfused int32 epilogue m=8 n=4096 k=4096")
    rc, _, _ = _linear_without_workspace(x.to(cuda), wp, torch.from_numpy(sw).to(cuda), None, n,
                                         _lib.EPI_I32, torch.int32)
    assert rc == _lib.ERR_WORKSPACE


def test_fused_path_strided_rows_and_fallbacks(cuda):
    from nanopointllm_amd import w8a8

    n, k = 48, 512
    _, qw, sw = weight_q(n, k, seed=12)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt = torch.from_numpy(sw).to(cuda)
    g = torch.Generator().manual_seed(1)
    big = torch.randn(6, 2 * k + 8, generator=g).to(torch.float16)
    cases = {
        "ld 1032 aligned": big[:, :k],            # fused, leading dimension 1032
        "unaligned base": big[:, 1:k + 1],        # not 16-byte aligned: quant + GEMV
    }
    for name, xv in cases.items():
        note(f"fused strided {name}")
        y = w8a8.linear_dynamic(big.to(cuda)[:, :k] if name == "ld 1032 aligned"
                                else big.to(cuda)[:, 1:k + 1], wp, swt, None, n)
        exp, _, _, _ = O.w8a8_linear_dynamic(xv.float().numpy(), qw, sw)
        np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


@pytest.mark.parametrize("m,n,k", [(3, 16 * 64 * 256, 128), (8, 16 * 64 * 256 + 32, 64),
                                   (5, 16 * 256 * 5, 2000), (8, 8192, 11008)])
def test_fused_decode_many_blocks_silu_bias(cuda, m, n, k):
    """Decode kernel with many 16-row output blocks per workgroup (64 on a
    256-CU device at the first shape) and K in several chunks per wavefront,
    through the SiLU*mul epilogue with a bias and the int32 epilogue.  The
    second shape is just past the fused kernel's block limit on a 256-CU
    device and runs quantization + GEMV instead; both must agree with the
    oracle."""
    from nanopointllm_amd import _lib, w8a8

    g = torch.Generator().manual_seed(n + k)
    x = (torch.randn(m, k, generator=g) * 3).to(torch.float16)
    _, q, s = weight_q(n, k, seed=k + 5)        # rows 2c / 2c+1 = gate / up of column c
    bias = np.linspace(-1.5, 1.5, n).astype(np.float32)
    wp = w8a8.pack_rows(torch.from_numpy(q).to(cuda))
    sw = torch.from_numpy(s).to(cuda)
    xc = x.to(cuda)
    note(f"fused many blocks m={m} n={n} k={k}")
    rc, _, _ = _linear_without_workspace(xc, wp, sw, None, n, _lib.EPI_I32, torch.int32)
    assert (rc == 0) == (n <= 16 * 64 * 256), "fused path taken iff within the block limit"
    acc = w8a8.linear_dynamic(xc, wp, sw, None, n, epilogue=_lib.EPI_I32).cpu().numpy()
    h = f16_to_np(w8a8.linear_dynamic(xc, wp, sw, torch.from_numpy(bias).to(cuda), n,
                                      epilogue=_lib.EPI_SILU_MUL))
    xq, sx = O.dynamic_per_token_quant(x.float().numpy())
    eacc = O.int32_matmul_f64(xq, q)
    np.testing.assert_array_equal(acc, eacc)
    eh = O.gateup_silu_mul_from_acc(eacc, sx, s, bias, layout="interleave")
    ulps = _fp16_ulps(h, eh)
    note(f"fused many blocks: exact {np.mean(ulps == 0):.6f}, max ulp {ulps.max()}")
    assert ulps.max() == 0


@pytest.mark.parametrize("m", [8, 200])
def test_linear_other_dtypes(cuda, m):
    from nanopointllm_amd import w8a8

    n, k = 96, 256
    g = torch.Generator().manual_seed(m)
    _, qw, sw = weight_q(n, k, seed=9)
    wp = w8a8.pack_rows(torch.from_numpy(qw).to(cuda))
    swt = torch.from_numpy(sw).to(cuda)
    xb = (torch.randn(m, k, generator=g) * 4).to(torch.bfloat16)
    note(f"linear bf16->bf16/f32 m={m}")
    exp, _ = _expected_linear(xb, qw, sw)
    yb = w8a8.linear_dynamic(xb.to(cuda), wp, swt, None, n)
    np.testing.assert_array_equal(bf16_bits(yb), O.f32_to_bf16_bits(exp))
    yf = w8a8.linear_dynamic(xb.to(cuda), wp, swt, None, n, out_dtype=torch.float32)
    np.testing.assert_array_equal(yf.cpu().numpy(), exp)
    xf = torch.randn(m, k, generator=g)
    note(f"linear f32 in m={m}")
    expf, _ = _expected_linear(xf, qw, sw)
    yf2 = w8a8.linear_dynamic(xf.to(cuda), wp, swt, None, n, out_dtype=torch.float32)
    np.testing.assert_array_equal(yf2.cpu().numpy(), expf)


def test_linear_3d_and_empty(cuda):
    from nanopointllm_amd import linear

    g = torch.Generator().manual_seed(2)
    w = torch.randn(32, 64, generator=g).to(torch.float16)
    lin = linear.W8A8Linear(linear.PackedW8A8Weight.from_float(w.to(cuda)))
    x = torch.randn(1, 5, 64, generator=g).to(torch.float16)
    note("linear 3d + empty")
    y = lin(x.to(cuda))
    assert y.shape == (1, 5, 32)
    _, qw, sw = O.per_output_weight_qdq(w.float().numpy())
    exp, _ = _expected_linear(x[0], qw, sw)
    np.testing.assert_array_equal(f16_to_np(y[0]), exp.astype(np.float16))
    assert lin(torch.empty(0, 64, dtype=torch.float16, device=cuda)).shape == (0, 32)


@pytest.mark.parametrize("m", [1, 8, 16, 64, 100, 567])
def test_linear_i8in_exact(cuda, m):
    from nanopointllm_amd import w8a8

    n, k = 80, 11008 if m <= 16 else 704
    xq = rand_i8((m, k), m)
    sx = O.scale_from_absmax(np.abs(np.random.default_rng(m).standard_normal((m, 1))) * 3)
    _, qw, sw = weight_q(n, k, seed=5)
    note(f"linear_i8in m={m} k={k}")
    y = w8a8.linear_i8in(xq.to(cuda), torch.from_numpy(sx).to(cuda),
                         w8a8.pack_rows(torch.from_numpy(qw).to(cuda)),
                         torch.from_numpy(sw).to(cuda), None, n, out_dtype=torch.float16)
    exp, _ = O.linear_from_quantized(xq.numpy(), sx, qw, sw)
    np.testing.assert_array_equal(f16_to_np(y), exp.astype(np.float16))


def test_integer_linear_per_output_kat_and_random(cuda):
    from nanopointllm_amd import w8a8

    kat = GOLDEN["tiny_int32_linear"]
    x = torch.tensor(kat["values"])
    w = torch.tensor(kat["weight"])
    b = torch.tensor(kat["bias"])
    s = torch.tensor(O.static_activation_scale(np.abs(x.numpy()).max()))
    note("integer_linear_per_output KAT")
    out, acc = w8a8.integer_linear_per_output(x.to(cuda), w.to(cuda),
                                              activation_scale=s.to(cuda), bias=b.to(cuda))
    eout, eacc = O.integer_linear_per_output(x.numpy(), w.numpy(), activation_scale=s.numpy(),
                                             bias=b.numpy())
    assert acc.dtype == torch.int32
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(out.cpu().numpy(), eout)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(9, 300, generator=g)
    w = torch.randn(70, 300, generator=g)
    s = torch.tensor(O.scale_from_absmax(np.abs(x.numpy()).max(1, keepdims=True)))
    note("integer_linear_per_output per-token")
    out, acc = w8a8.integer_linear_per_output(x.to(cuda), w.to(cuda), activation_scale=s.to(cuda))
    eout, eacc = O.integer_linear_per_output(x.numpy(), w.numpy(), activation_scale=s.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), eacc)
    np.testing.assert_array_equal(out.cpu().numpy(), eout)


# --------------------------------------------------------- gate/up + SiLU
def _gateup_case(m, inter, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, k, generator=g) * 1.5).to(torch.float16)
    wg = (torch.randn(inter, k, generator=g) * 0.05).to(torch.float16)
    wu = (torch.randn(inter, k, generator=g) * 0.05).to(torch.float16)
    return x, wg, wu


def _fp16_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in binary16 ulps (ordered-integer difference)."""
    def key(v):
        i = v.astype(np.float16).view(np.int16).astype(np.int32)
        return np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("m", [1, 8, 16, 64, 65, 567])
def test_gateup_silu_mul(cuda, m):
    from nanopointllm_amd import linear

    inter, k = 264, 512
    x, wg, wu = _gateup_case(m, inter, k, seed=m)
    gate = torch.nn.Linear(k, inter, bias=False)
    up = torch.nn.Linear(k, inter, bias=False)
    gate.weight.data, up.weight.data = wg.to(cuda), wu.to(cuda)
    mod = linear.W8A8GateUpSiluMul(gate, up)
    note(f"gateup silu m={m}")
    h = f16_to_np(mod(x.to(cuda)))
    acc = mod.accumulators(x.to(cuda)).cpu().numpy()
    _, qg, sg = O.per_output_weight_qdq(wg.float().numpy())
    _, qu, su = O.per_output_weight_qdq(wu.float().numpy())
    qp = O.pack_gateup_rows(qg, qu, "interleave")
    sp = O.pack_gateup_rows(sg[:, None], su[:, None], "interleave")[:, 0]
    xq, sx = O.dynamic_per_token_quant(x.float().numpy())
    eacc = O.int32_matmul_f64(xq, qp)
    np.testing.assert_array_equal(acc, eacc)
    eh = O.gateup_silu_mul_from_acc(eacc, sx, sp, layout="interleave")
    ulps = _fp16_ulps(h, eh)
    note(f"gateup silu m={m}: exact {np.mean(ulps == 0):.6f}, max ulp {ulps.max()}")
    assert ulps.max() == 0


@pytest.mark.parametrize("m", [8, 567])
def test_mlp_int8_chain(cuda, m):
    """gate/up -> SiLU*mul -> static int8 requant -> int8-in down projection."""
    from nanopointllm_amd import linear, w8a8

    inter, k = 264, 512
    x, wg, wu = _gateup_case(m, inter, k, seed=100 + m)
    g = torch.Generator().manual_seed(7)
    wd = (torch.randn(k, inter, generator=g) * 0.05).to(torch.float16)
    mods = [torch.nn.Linear(k, inter, bias=False), torch.nn.Linear(k, inter, bias=False),
            torch.nn.Linear(inter, k, bias=False)]
    for mod_, wt in zip(mods, (wg, wu, wd)):
        mod_.weight.data = wt.to(cuda)
    h_ref = linear.W8A8GateUpSiluMul(mods[0], mods[1])(x.to(cuda))
    h_scale = float(O.static_activation_scale(float(h_ref.abs().max().item())))
    mlp = linear.W8A8MLP(*mods, h_scale=h_scale)
    note(f"mlp int8 chain m={m}")
    hq = mlp.gate_up.forward_q8(x.to(cuda), h_scale).cpu().numpy()
    y = f16_to_np(mlp(x.to(cuda)))
    # Stage 1: the int8 epilogue equals the oracle's requant of the GPU's own h.
    eq = O.quantize_symmetric(f16_to_np(h_ref).astype(np.float32), np.float32(h_scale))
    np.testing.assert_array_equal(hq, eq)
    # Stage 2: the down projection on the GPU's int8 h is exact.
    _, qd, sd = O.per_output_weight_qdq(wd.float().numpy())
    sx = np.full((m, 1), h_scale, np.float32)
    exp, _ = O.linear_from_quantized(hq, sx, qd, sd)
    np.testing.assert_array_equal(y, exp.astype(np.float16))
    acc = w8a8.gemm_i32(torch.from_numpy(hq).to(cuda), mlp.down.weight_q.packed, k)
    np.testing.assert_array_equal(acc.cpu().numpy(), O.int32_matmul_f64(hq, qd))


def test_packed_qkv_split_matches_separate_linears(cuda):
    from nanopointllm_amd import linear

    g = torch.Generator().manual_seed(11)
    k, heads, hd = 256, 4, 32
    projs = []
    for _ in range(3):
        p = torch.nn.Linear(k, heads * hd, bias=True)
        p.weight.data = (torch.randn(heads * hd, k, generator=g) * 0.05).to(torch.float16).to(cuda)
        p.bias.data = torch.randn(heads * hd, generator=g).to(torch.float16).to(cuda)
        projs.append(p)
    qkv = linear.W8A8PackedQKV(*projs, num_heads=heads, num_kv_heads=heads, head_dim=hd)
    x = torch.randn(1, 6, k, generator=g).to(torch.float16)
    note("packed qkv")
    q, kk, v = qkv.project(x.to(cuda))
    for got, p in zip((q, kk, v), projs):
        sep = linear.W8A8Linear.from_linear(p)(x[0].to(cuda))
        np.testing.assert_array_equal(f16_to_np(got.reshape(6, -1)), f16_to_np(sep))


# ----------------------------------------------------- full LLaMA-7B shapes
@pytest.mark.parametrize("m", [1, 8, 560])
@pytest.mark.parametrize("proj", ["qkv", "o", "gateup", "down"])
def test_llama7b_shapes_exact(cuda, m, proj):
    from nanopointllm_amd import w8a8
    import workloads as W

    spec = {p.name: p for p in W.PROJECTIONS}[proj]
    x = (W.decode_activations(m, spec.k, seed=m) if m <= 16
         else W.prefill_activations(m, spec.k, seed=m))
    wq = torch.randint(-127, 128, (spec.n, spec.k), generator=torch.Generator().manual_seed(3),
                       dtype=torch.int8)
    sw = O.scale_from_absmax(np.abs(np.random.default_rng(1).standard_normal(spec.n)) * 0.08)
    note(f"llama7b {proj} m={m} n={spec.n} k={spec.k}")
    wp = w8a8.pack_rows(wq.to(cuda))
    xc = x.to(cuda)
    acc = w8a8.linear_dynamic(xc, wp, torch.from_numpy(sw).to(cuda), None, spec.n,
                              epilogue=0).cpu().numpy()
    xq, sx = O.dynamic_per_token_quant(x.float().numpy())
    eacc = O.int32_matmul_f64(xq, wq.numpy())
    np.testing.assert_array_equal(acc, eacc)
    if not spec.silu:
        y = w8a8.linear_dynamic(xc, wp, torch.from_numpy(sw).to(cuda), None, spec.n)
        np.testing.assert_array_equal(f16_to_np(y), O.dequant_epilogue(eacc, sx, sw).astype(np.float16))
