"""Fused activation prologue: residual add -> RMSNorm -> SmoothQuant divide ->
int8 quantization, in one kernel per row (w8a8_prologue_quant).

Bars: the residual add, the smooth divide and the quantization are bit-exact
against the oracle.  RMSNorm is bit-exact where the binary32 sum of squares is
exact in any order; on general inputs the normalized rows are within one
16-bit ulp of the oracle (>= 99.9% bit-equal) because the kernel and torch's
CPU ``mean`` sum in different orders, and the quantization of the kernel's own
normalized rows is bit-exact.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu

TDT = {"f16": torch.float16, "bf16": torch.bfloat16}


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _rand16(shape, seed, dtype, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    x[..., : min(5, shape[-1])] *= 40
    return x.to(TDT[dtype])


def _ulps(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(TDT[dtype]).view(torch.int16)
    u = torch.from_numpy(np.ascontiguousarray(b, np.float32)).to(TDT[dtype]).view(torch.int16)
    key = lambda i: torch.where(i < 0, -(i.int() & 0x7FFF), i.int())
    return (key(t) - key(u)).abs().numpy()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("m,k", [(1, 4096), (8, 4096), (3, 11008), (300, 1000), (2, 32768), (5, 7)])
def test_residual_add_and_per_token_quant_exact(cuda, dtype, m, k):
    from nanopointllm_amd import w8a8

    x, r = _rand16((m, k), m + k, dtype), _rand16((m, k), 2 * k + m, dtype, 0.05)
    note(f"prologue residual {dtype} m={m} k={k}")
    out = w8a8.prologue_quant(x.to(cuda), residual=r.to(cuda), return_rows=True)
    summed = O.residual_add(x.float().numpy(), r.float().numpy(), dtype)
    np.testing.assert_array_equal(out.residual.float().cpu().numpy(), summed)
    np.testing.assert_array_equal(out.rows.float().cpu().numpy(), summed)
    eq, es = O.dynamic_per_token_quant(summed)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), es[:, 0])
    np.testing.assert_array_equal(out.q.cpu().numpy(), eq)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_smoothquant_divide_dynamic_and_static_exact(cuda, dtype):
    from nanopointllm_amd import w8a8

    m, k = 6, 3000
    x = _rand16((m, k), 5, dtype)
    g = torch.Generator().manual_seed(6)
    smooth = torch.exp(torch.rand(k, generator=g) * 6 - 3).to(TDT[dtype])
    note(f"smoothquant {dtype}")
    xs = O.smooth_divide(x.float().numpy(), smooth.float().numpy(), dtype)
    qdq, s = w8a8.smoothquant_activation_qdq(x.to(cuda), smooth.to(cuda))
    eq, es = O.dynamic_per_token_quant(xs)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(qdq.float().cpu().numpy(),
                                  O.round16(eq.astype(np.float32) * es, dtype))
    static = O.static_activation_scale(np.abs(xs).max() * 0.5)          # clips some values
    out = w8a8.prologue_quant(x.to(cuda), smooth=smooth.to(cuda),
                              static_scale=float(static))
    np.testing.assert_array_equal(out.q.cpu().numpy(), O.quantize_symmetric(xs, static))


def _exact_sum_rows(m, k, seed, dtype):
    """Rows of multiples of 1/8 in [-4, 4]: every binary32 partial sum of their
    squares is exact, so the sum does not depend on its order."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-32, 33, (m, k), generator=g).float() / 8).to(TDT[dtype])


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("m,k", [(1, 4096), (8, 4096), (4, 5120), (64, 512)])
def test_rmsnorm_quant_exact_where_the_sum_is_exact(cuda, dtype, m, k):
    from nanopointllm_amd import w8a8

    x = _exact_sum_rows(m, k, m * 7 + k, dtype)
    x[:, 3] = -0.0   # normalizes to -0, as torch's x * rsqrt(...) and w * x do
    w = _rand16((k,), k, dtype, 0.5).abs() + 0.25
    w = w.to(TDT[dtype])
    note(f"rmsnorm exact-sum {dtype} m={m} k={k}")
    out = w8a8.prologue_quant(x.to(cuda), norm_weight=w.to(cuda), eps=1e-6, return_rows=True)
    y = O.rmsnorm(x.float().numpy(), w.float().numpy(), 1e-6, dtype)
    rows = out.rows.float().cpu().numpy()
    np.testing.assert_array_equal(rows, y)
    np.testing.assert_array_equal(np.signbit(rows), np.signbit(y))
    eq, es = O.dynamic_per_token_quant(y)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), es[:, 0])
    np.testing.assert_array_equal(out.q.cpu().numpy(), eq)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("weight_f32", [False, True])
def test_rmsnorm_residual_smooth_quant_general_inputs(cuda, dtype, weight_f32):
    from nanopointllm_amd import w8a8

    m, k = 16, 4096
    x, r = _rand16((m, k), 21, dtype), _rand16((m, k), 22, dtype, 0.1)
    g = torch.Generator().manual_seed(23)
    w = torch.rand(k, generator=g) + 0.5
    w = w if weight_f32 else w.to(TDT[dtype])
    smooth = (torch.rand(k, generator=g) + 0.5).to(TDT[dtype])
    note(f"rmsnorm general {dtype} f32 weight={weight_f32}")
    out = w8a8.prologue_quant(x.to(cuda), residual=r.to(cuda), norm_weight=w.to(cuda),
                              eps=1e-5, smooth=smooth.to(cuda), return_rows=True)
    summed = O.residual_add(x.float().numpy(), r.float().numpy(), dtype)
    np.testing.assert_array_equal(out.residual.float().cpu().numpy(), summed)
    y = O.rmsnorm(summed, w.float().numpy(), 1e-5, dtype, weight_f32=weight_f32)
    y = O.smooth_divide(y, smooth.float().numpy(), None if weight_f32 else dtype)
    rows = out.rows.float().cpu().numpy()
    assert out.rows.dtype == (torch.float32 if weight_f32 else TDT[dtype])
    if weight_f32:
        # rows = w * xn with xn rounded to the 16-bit dtype: a flip of xn by
        # one ulp moves the row by at most one 16-bit ulp, relatively.
        ulp16 = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7
        rel = np.abs(rows - y) / np.maximum(np.abs(y), 1e-30)
        assert rel.max() <= ulp16 and np.mean(rows == y) > 0.999
    else:
        d = _ulps(rows, y, dtype)
        note(f"rmsnorm general: exact {np.mean(d == 0):.6f}, max ulp {d.max()}")
        assert d.max() <= 1 and np.mean(d == 0) > 0.999
    # stage-wise: the quantization of the kernel's own rows is bit-exact
    eq, es = O.dynamic_per_token_quant(rows)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), es[:, 0])
    np.testing.assert_array_equal(out.q.cpu().numpy(), eq)


def test_prologue_rejects_bad_arguments(cuda):
    from nanopointllm_amd import w8a8

    x = torch.zeros(2, 64, dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        w8a8.prologue_quant(x.float())
    with pytest.raises(ValueError, match="one value per hidden channel"):
        w8a8.prologue_quant(x, norm_weight=torch.ones(63, device=cuda, dtype=torch.float16))
    with pytest.raises(ValueError, match="positive"):
        w8a8.prologue_quant(x, static_scale=0.0)
    with pytest.raises(ValueError):
        w8a8.prologue_quant(torch.zeros(1, 40000, dtype=torch.float16, device=cuda))


class _Norm(torch.nn.Module):
    def __init__(self, hidden, dtype, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.weight = torch.nn.Parameter((torch.rand(hidden, generator=g) + 0.5).to(dtype))
        self.variance_epsilon = 1e-6


def test_rmsnorm_packed_qkv_decode_matches_staged_path(cuda):
    """One fused norm+quant kernel + int8-in QKV equals RMSNorm rows quantized
    by the linear itself, and stays within the reference test's tolerance of
    the dense fp32 computation (tests/test_paged_attention.py:316-357)."""
    from nanopointllm_amd import inject, linear, w8a8

    H, Hkv, D = 8, 4, 64
    hidden = H * D
    g = torch.Generator().manual_seed(9)
    projs = [torch.nn.Linear(hidden, n, bias=False) for n in (H * D, Hkv * D, Hkv * D)]
    for p in projs:
        p.weight.data = (torch.randn(p.weight.shape, generator=g) * 0.02).to(torch.float16)
        p.to(cuda)
    qkv = linear.W8A8PackedQKV(*projs, num_heads=H, num_kv_heads=Hkv, head_dim=D)
    norm = _Norm(hidden, torch.float16, 10).to(cuda)
    hs = (torch.randn(1, 5, hidden, generator=g)).to(torch.float16).to(cuda)
    note("rmsnorm_packed_qkv_decode")
    q, k, v = inject.rmsnorm_packed_qkv_decode(hs, norm, qkv)
    rows = w8a8.prologue_quant(hs[0], norm_weight=norm.weight, eps=1e-6, return_rows=True).rows
    q2, k2, v2 = qkv.project(rows)
    for a, b in ((q, q2), (k, k2), (v, v2)):
        assert torch.equal(a, b)
    x = hs[0].float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    x = (norm.weight.float() * x)
    ref = torch.cat([x @ p.weight.float().t() for p in projs], -1)
    got = torch.cat([q.reshape(5, -1), k.reshape(5, -1), v.reshape(5, -1)], -1).float()
    torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("h_scale", [None, 0.05])
def test_residual_rmsnorm_mlp_decode_matches_module_path(cuda, h_scale):
    from nanopointllm_amd import inject, linear, w8a8

    hidden, inter = 256, 384
    g = torch.Generator().manual_seed(12)
    mk = lambda o, i: torch.nn.Linear(i, o, bias=False)
    gate, up, down = mk(inter, hidden), mk(inter, hidden), mk(hidden, inter)
    for p in (gate, up, down):
        p.weight.data = (torch.randn(p.weight.shape, generator=g) * 0.05).to(torch.float16)
        p.to(cuda)
    mlp = linear.W8A8MLP(gate, up, down, h_scale=h_scale)
    norm = _Norm(hidden, torch.float16, 13).to(cuda)
    hs = torch.randn(1, 4, hidden, generator=g).to(torch.float16).to(cuda)
    res = torch.randn(1, 4, hidden, generator=g).to(torch.float16).to(cuda)
    note(f"residual_rmsnorm_mlp_decode h_scale={h_scale}")
    summed, out = inject.residual_rmsnorm_mlp_decode(hs, res, norm, mlp)
    assert summed.shape == (1, 4, hidden) and out.shape == (1, 4, hidden)
    np.testing.assert_array_equal(summed[0].float().cpu().numpy(),
                                  O.residual_add(hs[0].float().cpu().numpy(),
                                                 res[0].float().cpu().numpy(), "f16"))
    rows = w8a8.prologue_quant(summed[0], norm_weight=norm.weight, eps=1e-6,
                               return_rows=True).rows
    assert torch.equal(out[0], mlp(rows))
