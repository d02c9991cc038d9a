"""Pins the CPU oracle (oracle/w8a8_oracle.py) before it is trusted.

Every check here is independent of the oracle's own formula: reference
known-answer vectors (tests/golden/reference_vectors.json), exact rational
arithmetic (``fractions.Fraction`` with an explicit round-to-nearest-even
helper), brute force over every binary16 value, closed forms, and torch's own
float64 -> bfloat16 conversion.  A few "planted mistake" tests show the pins
reject plausible bugs.
"""
from __future__ import annotations

import json
import math
import random
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import w8a8_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


# ----------------------------------------------------------- exact helpers
def round_binary(value: Fraction, mant_bits: int, emin: int) -> Fraction:
    """Round a rational to nearest-even in a binary format with `mant_bits`
    significand bits, minimum normal exponent `emin` and gradual underflow."""
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    a = abs(value)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - mant_bits + 1)
    return sign * round(a / quantum) * quantum


def r32(v) -> Fraction:
    return round_binary(Fraction(v), 24, -126)


def r16(v) -> Fraction:
    return round_binary(Fraction(v), 11, -14)


def rbf16(v) -> Fraction:
    return round_binary(Fraction(v), 8, -126)


TINY = Fraction(1, 2 ** 14)


def exact_scale(absmax) -> Fraction:
    return max(r16(r32(max(Fraction(absmax), TINY) / 127)), TINY)


def exact_quant(x, s) -> int:
    q = round(r32(Fraction(x) / Fraction(s)))
    return max(-127, min(127, q))


def all_finite_fp16() -> np.ndarray:
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return v[np.isfinite(v)]


# ---------------------------------------------------------- quantization
def test_reference_rounding_clipping_kat():
    kat = GOLDEN["rounding_clipping"]
    q = O.quantize_symmetric(np.array(kat["values"], np.float32), np.float32(kat["scale"]))
    assert q.dtype == np.int8
    assert q.tolist() == kat["asserted"]


def test_quantize_rejects_nonpositive_scale():
    with pytest.raises(ValueError, match="positive"):
        O.quantize_symmetric(np.ones(1), np.float32(0.0))
    with pytest.raises(ValueError, match="positive"):
        O.quantize_symmetric(np.ones((2, 1)), np.array([[1.0], [-1.0]], np.float32))


@pytest.mark.parametrize("scale", [2.0 ** -14, 0.0124359130859375, 1.0 / 127, 0.5, 1.0, 3.140625])
def test_quantize_brute_force_all_fp16(scale):
    s = np.float32(np.float16(scale))
    xs = all_finite_fp16()
    got = O.quantize_symmetric(xs, s)
    # For binary16 inputs the exact quotient is never within 2**-13 of a
    # half-integer unless it is one, so rounding the exact rational agrees
    # with rounding the binary32 quotient.
    sf = Fraction(float(s))
    exp = np.array([max(-127, min(127, round(Fraction(float(x)) / sf))) for x in xs], np.int8)
    np.testing.assert_array_equal(got, exp)


def test_quantize_binary32_inputs_match_rational_division():
    rng = np.random.default_rng(11)
    xs = (rng.standard_normal(3000) * rng.choice([1e-3, 1.0, 30.0], 3000)).astype(np.float32)
    for s in (np.float32(np.float16(0.0124359)), np.float32(np.float16(0.2))):
        got = O.quantize_symmetric(xs, s)
        exp = [exact_quant(float(x), float(s)) for x in xs]
        assert got.tolist() == exp


def test_scale_from_absmax_special_and_random():
    specials = [0.0, 1e-30, 2.0 ** -14, 127 * 2.0 ** -14, 127 * 2.0 ** -14 * 1.01, 0.5, 1.0,
                4.0, 40.0, 127.0, 1000.0, 65504.0 * 127 * 0.5]
    rng = np.random.default_rng(5)
    rand = (np.abs(rng.standard_normal(2000)) * rng.choice([1e-4, 1e-2, 1.0, 50.0], 2000))
    values = np.concatenate([np.array(specials), rand]).astype(np.float32)
    got = O.scale_from_absmax(values)
    exp = np.array([float(exact_scale(float(v))) for v in values], np.float32)
    np.testing.assert_array_equal(got, exp)
    assert got[0] == np.float32(2.0 ** -14)   # all-zero row -> 2**-14
    assert np.all(got >= np.float32(2.0 ** -14))


def test_dynamic_per_token_scale_shape_kat():
    kat = GOLDEN["per_token_scale_shape"]
    v = np.array(kat["values"], np.float32)
    qdq, scales = O.dynamic_per_token_activation_qdq(v)
    assert list(scales.shape) == kat["asserted_dynamic_scale_shape"]
    static = O.quantize_symmetric(v, O.static_activation_scale(np.abs(v).max())).astype(np.float32)
    static = static * O.static_activation_scale(np.abs(v).max())
    assert np.mean((qdq - v) ** 2) < np.mean((static - v) ** 2)


def test_per_output_weight_rows_are_independent_quantizations():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((5, 259)).astype(np.float32)
    deq, q, s = O.per_output_weight_qdq(w)
    assert q.shape == w.shape and s.shape == (5,)
    for r in range(5):
        sr = exact_scale(float(np.abs(w[r]).max()))
        assert s[r] == np.float32(float(sr))
        assert q[r].tolist() == [exact_quant(float(x), float(sr)) for x in w[r]]
    np.testing.assert_array_equal(deq, (q.astype(np.float32) * s[:, None]))


def test_per_row_quant_commutes_with_row_packing():
    rng = np.random.default_rng(9)
    wg, wu = (rng.standard_normal((6, 64)).astype(np.float32) for _ in range(2))
    _, qg, sg = O.per_output_weight_qdq(wg)
    _, qu, su = O.per_output_weight_qdq(wu)
    for layout in ("split", "interleave"):
        _, qp, sp = O.per_output_weight_qdq(O.pack_gateup_rows(wg, wu, layout))
        np.testing.assert_array_equal(qp, O.pack_gateup_rows(qg, qu, layout))
        np.testing.assert_array_equal(sp, O.pack_gateup_rows(sg[:, None], su[:, None], layout)[:, 0])


# ----------------------------------------------------------- int32 product
def test_package_fixture_integer_golden():
    pkg = GOLDEN["package"]
    a = np.array(pkg["activation"], np.int8)
    w = np.array(pkg["weight"], np.int8)
    exp = np.array(pkg["derived_integer_golden"], np.int32)
    np.testing.assert_array_equal(O.int32_matmul_f64(a, w), exp)
    np.testing.assert_array_equal(O.int32_matmul_int(a, w), exp)


def test_dense64_caller_owned_int8_fixture():
    fx = GOLDEN["dense64_caller_int8"]
    m, n, k = fx["m"], fx["n"], fx["k"]
    a = ((np.arange(m * k) * 7 + 3) % 255 - 127).astype(np.int8).reshape(m, k)
    w = ((np.arange(n * k) * 11 + 5) % 255 - 127).astype(np.int8).reshape(n, k)
    brute = [[sum(int(a[i, t]) * int(w[j, t]) for t in range(k)) for j in range(n)] for i in range(m)]
    np.testing.assert_array_equal(O.int32_matmul_f64(a, w), np.array(brute, np.int32))


def test_int32_formulations_agree_and_hit_extremes():
    rng = np.random.default_rng(1)
    a = rng.integers(-127, 128, (7, 700), dtype=np.int8)
    w = rng.integers(-127, 128, (9, 700), dtype=np.int8)
    np.testing.assert_array_equal(O.int32_matmul_f64(a, w), O.int32_matmul_int(a, w))
    k = 133144  # largest K with K * 127**2 < 2**31
    full = np.full((1, k), 127, np.int8)
    assert int(O.int32_matmul_f64(full, -full)[0, 0]) == -k * 127 * 127
    with pytest.raises(OverflowError):
        O.int32_matmul_f64(np.ones((1, k + 1), np.int8), np.ones((1, k + 1), np.int8))


def test_dequant_epilogue_matches_rational_rounding_chain():
    rng = np.random.default_rng(3)
    acc = rng.integers(-177_000_000, 177_000_000, (6, 40)).astype(np.int32)
    acc[0, :4] = [0, 1, -1, 16777217]  # 2**24 + 1 is not binary32-representable
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((6, 1))) * 5)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(40)) * 0.05)
    bias = rng.standard_normal(40).astype(np.float32)
    got = O.dequant_epilogue(acc, sx, sw, bias)
    for i in range(6):
        for j in range(40):
            v = r32(int(acc[i, j]))
            v = r32(v * Fraction(float(sx[i, 0])))
            v = r32(v * Fraction(float(sw[j])))
            v = r32(v + Fraction(float(bias[j])))
            assert got[i, j] == np.float32(float(v))


def test_dequant_is_not_fma_contracted():
    # A planted mistake: one fused rounding (acc*sx*sw + b in float64, rounded
    # once) must differ from the reference's binary32 step chain somewhere.
    rng = np.random.default_rng(12)
    acc = rng.integers(-10_000_000, 10_000_000, (64, 64)).astype(np.int32)
    sx = O.scale_from_absmax(np.abs(rng.standard_normal((64, 1))) * 3)
    sw = O.scale_from_absmax(np.abs(rng.standard_normal(64)) * 0.05)
    bias = rng.standard_normal(64).astype(np.float32)
    fused = (acc.astype(np.float64) * sx * sw + bias).astype(np.float32)
    assert np.any(fused != O.dequant_epilogue(acc, sx, sw, bias))


def test_tiny_integer_linear_kat():
    kat = GOLDEN["tiny_int32_linear"]
    x = np.array(kat["values"], np.float32)
    w = np.array(kat["weight"], np.float32)
    b = np.array(kat["bias"], np.float32)
    s = O.static_activation_scale(np.abs(x).max())
    out, acc = O.integer_linear_per_output(x, w, activation_scale=s, bias=b)
    assert acc.dtype == np.int32 and out.shape == (1, 2)
    # QDQ then float64 linear, computed without the oracle's epilogue.
    qx = [exact_quant(float(v), float(s)) for v in x[0]]
    qdq_x = np.array(qx, np.float64) * float(s)
    qdq_w = []
    for row in w:
        sr = exact_scale(float(np.abs(row).max()))
        qdq_w.append([exact_quant(float(v), float(sr)) * float(sr) for v in row])
    ref = qdq_x @ np.array(qdq_w).T + b
    assert np.max(np.abs(out[0] - ref)) < kat["asserted_integer_vs_qdq_fp32_max_abs_below"]
    # int32 accumulators by hand: x/s and w/s_w quantize to exact multiples here.
    assert acc.tolist() == [[int(sum(qx[t] * exact_quant(float(w[j, t]),
                                                          float(exact_scale(float(np.abs(w[j]).max()))))
                                     for t in range(4))) for j in range(2)]]
    with pytest.raises(ValueError, match="shapes do not match"):
        O.integer_linear_per_output(x, w[:, :3], activation_scale=s)


def test_planted_truncating_quantizer_fails_kat():
    kat = GOLDEN["rounding_clipping"]
    v = np.array(kat["values"], np.float32)
    truncating = np.clip(np.trunc(v / np.float32(kat["scale"])), -127, 127).astype(np.int8)
    half_away = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127).astype(np.int8)
    assert truncating.tolist() != kat["asserted"]
    assert half_away.tolist() != kat["asserted"]


# ------------------------------------------------------------ SiLU * mul
@pytest.mark.parametrize("fn", ["silu_mul_hf", "silu_mul_closed_form"])
def test_silu_mul_within_one_binary16_ulp_of_float64(fn):
    g = np.linspace(-12, 12, 4001).astype(np.float16)
    u = np.tile(np.array([-3.5, -1.0, 0.25, 1.0, 7.75], np.float16), 801)[:4001]
    got = getattr(O, fn)(g, u).astype(np.float64)
    g64 = g.astype(np.float64)
    s64 = np.float16(g64 / (1.0 + np.exp(-g64))).astype(np.float64)
    exp = (s64 * u.astype(np.float64)).astype(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(exp).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - exp) <= ulp)


def test_gateup_layouts_pair_the_same_outputs():
    rng = np.random.default_rng(2)
    acc_g = rng.integers(-200000, 200000, (3, 8)).astype(np.int32)
    acc_u = rng.integers(-200000, 200000, (3, 8)).astype(np.int32)
    sx = np.full((3, 1), 0.01, np.float32)
    sg = np.full(8, 0.001, np.float32)
    su = np.full(8, 0.002, np.float32)
    split = O.gateup_silu_mul_from_acc(np.concatenate([acc_g, acc_u], 1), sx,
                                       np.concatenate([sg, su]), layout="split")
    inter = O.gateup_silu_mul_from_acc(np.stack([acc_g, acc_u], 2).reshape(3, 16), sx,
                                       np.stack([sg, su], 1).reshape(-1), layout="interleave")
    np.testing.assert_array_equal(split, inter)


# ------------------------------------------------------------- requant a17
def test_requant_locked_vectors():
    fx = GOLDEN["requant_locked"]
    outs = [O.requantize_int32(*v) for v in fx["vectors"]]
    assert outs[3:7] == fx["asserted_outputs_3_7"]
    assert outs[7:9] == fx["asserted_outputs_7_9"]
    for (acc, bias, mult, shift), got in zip(fx["vectors"], outs):
        exact = Fraction((acc + bias) * mult, 2 ** shift)
        assert got == max(-127, min(127, round(exact)))


def test_requant_scale_compiler():
    c = GOLDEN["requant_locked"]["asserted_compile"]
    mult, shift, ratio, rel = O.compile_fp16_requant_scale(
        c["activation_scale"], c["weight_scale"], c["output_scale"])
    assert 0 < mult < 2 ** 32 and 0 <= shift <= 63
    assert rel < c["relative_error_below"]
    half = lambda v: struct.unpack("e", struct.pack("e", v))[0]
    assert ratio == half(c["activation_scale"]) * half(c["weight_scale"]) / half(c["output_scale"])
    with pytest.raises(ValueError):
        O.compile_requant_ratio(0.0)


# -------------------------------------------------------- bf16 dequant a18
def _fp16_bits_value(bits: int) -> Fraction:
    return Fraction(struct.unpack("<e", struct.pack("<H", bits))[0])


def test_bf16_dequant_locked_vectors():
    fx = GOLDEN["bf16_dequant_locked"]
    outs = [O.dequantize_int32_to_bf16(*v) for v in fx["vectors"]]
    assert outs[0:3] == fx["asserted_outputs_0_3"]
    assert outs[6] == fx["asserted_output_6"]
    for (acc, sa, sw), got in zip(fx["vectors"], outs):
        exact = acc * _fp16_bits_value(sa) * _fp16_bits_value(sw)
        v = rbf16(exact)
        if abs(v) >= Fraction(2) ** 128:
            exp = (0x8000 if v < 0 else 0) | 0x7F80
        else:
            exp = int(O.f32_to_bf16_bits(np.float32(float(v)))) if v != 0 else (
                0x8000 if exact < 0 else 0)
        assert got == exp


def test_bf16_dequant_random_vs_torch_float64():
    torch = pytest.importorskip("torch")
    gen = random.Random(GOLDEN["bf16_dequant_locked"]["random_check"]["seed"])
    for _ in range(GOLDEN["bf16_dequant_locked"]["random_check"]["count"]):
        acc = gen.randint(-(1 << 31), (1 << 31) - 1)
        sa = gen.randrange(0x0001, 0x7C00) | (gen.randrange(2) << 15)
        sw = gen.randrange(0x0001, 0x7C00) | (gen.randrange(2) << 15)
        va = struct.unpack("e", struct.pack("H", sa))[0]
        vw = struct.unpack("e", struct.pack("H", sw))[0]
        exp = int(torch.tensor(acc * va * vw, dtype=torch.float64)
                  .to(torch.bfloat16).view(torch.uint16).item())
        assert O.dequantize_int32_to_bf16(acc, sa, sw) == exp


def test_bf16_rounding_helper_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    v = rng.standard_normal(5000).astype(np.float32) * 1e3
    u = v.view(np.uint32).copy()
    u[:100] = (u[:100] & 0xFFFF0000) | 0x8000   # exact ties
    v = u.view(np.float32)
    exp = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(v), exp)


# ------------------------------------------------------------- packing a12
def test_qkv_and_gateup_row_packing():
    wq, wk, wv = (np.full((4, 3), i, np.int8) for i in (1, 2, 3))
    assert O.pack_qkv_rows(wq, wk, wv)[:, 0].tolist() == [1] * 4 + [2] * 4 + [3] * 4
    wg = np.arange(3)[:, None].repeat(2, 1)
    wu = 10 + np.arange(3)[:, None].repeat(2, 1)
    assert O.pack_gateup_rows(wg, wu, "interleave")[:, 0].tolist() == [0, 10, 1, 11, 2, 12]
    assert O.pack_gateup_rows(wg, wu, "split")[:, 0].tolist() == [0, 1, 2, 10, 11, 12]
    with pytest.raises(ValueError):
        O.pack_gateup_rows(wg, wu, "bogus")


def test_tensor_error_metrics():
    ref = np.array([1.0, -2.0, 0.0], np.float32)
    cand = np.array([1.5, -2.0, 1e-9], np.float32)
    e = O.tensor_error(ref, cand)
    assert math.isclose(e["max_abs"], 0.5)
    assert math.isclose(e["mean_abs"], (0.5 + 1e-9) / 3, rel_tol=1e-6)


# ------------------------------------------------ activation prologue (f3/f4)
def _ulp_distance16(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """|a - b| in units in the last place of the 16-bit dtype (values are
    exactly representable in it)."""
    if dtype == "f16":
        ia = a.astype(np.float16).view(np.int16).astype(np.int64)
        ib = b.astype(np.float16).view(np.int16).astype(np.int64)
    else:
        ia = O.f32_to_bf16_bits(a).view(np.int16).astype(np.int64)
        ib = O.f32_to_bf16_bits(b).view(np.int16).astype(np.int64)
    key = lambda i: np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(key(ia) - key(ib))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_residual_add_and_smooth_divide_match_16bit_arithmetic(dtype):
    import torch

    rng = np.random.default_rng(1)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    a = torch.from_numpy(rng.standard_normal(5000).astype(np.float32) * 30).to(tdt)
    b = torch.from_numpy(rng.standard_normal(5000).astype(np.float32) * 0.01).to(tdt)
    s = torch.from_numpy(np.exp(rng.uniform(-5, 5, 5000)).astype(np.float32)).to(tdt)
    an, bn, sn = a.float().numpy(), b.float().numpy(), s.float().numpy()
    np.testing.assert_array_equal(O.residual_add(an, bn, dtype), (a + b).float().numpy())
    np.testing.assert_array_equal(O.smooth_divide(an, sn, dtype), (a / s).float().numpy())
    np.testing.assert_array_equal(O.smooth_divide(an, sn, None), (a.float() / s.float()).numpy())


def _rmsnorm_f64(x, w, eps, dtype):
    """Float64 closed form rounded once to the 16-bit dtype per step the
    reference rounds (x.to(dtype), then weight * x in dtype)."""
    x64 = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + eps)
    xn = O.round16((x64 * r).astype(np.float32), dtype)
    return O.round16(np.asarray(w, np.float64) * xn, dtype)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rmsnorm_within_one_ulp_of_float64_and_planted_mistakes_fail(dtype):
    rng = np.random.default_rng(2)
    x = O.round16(rng.standard_normal((6, 4096)).astype(np.float32) * 3, dtype)
    x[0, :8] *= 60
    w = O.round16(rng.uniform(0.2, 2.0, 4096).astype(np.float32), dtype)
    eps = 1e-6
    y = O.rmsnorm(x, w, eps, dtype)
    ref = _rmsnorm_f64(x, w, eps, dtype)
    # Only the binary32 rsqrt factor differs from the float64 chain, which
    # flips a 16-bit rounding on very few elements.
    assert _ulp_distance16(y, ref, dtype).max() <= 1
    assert np.mean(y == ref) > 0.999

    def eps_outside(x, w):
        x = np.asarray(x, np.float32)
        r = np.float32(1) / (np.sqrt(np.sum(x * x, -1, keepdims=True, dtype=np.float32)
                                     / np.float32(x.shape[-1])) + np.float32(eps))
        return O.round16(w * O.round16(x * r, dtype), dtype)

    def sum_not_mean(x, w):
        x = np.asarray(x, np.float32)
        r = np.float32(1) / np.sqrt(np.sum(x * x, -1, keepdims=True, dtype=np.float32)
                                    + np.float32(eps))
        return O.round16(w * O.round16(x * r, dtype), dtype)

    def weight_before_rounding(x, w):
        x = np.asarray(x, np.float32)
        r = np.float32(1) / np.sqrt(np.sum(x * x, -1, keepdims=True, dtype=np.float32)
                                    / np.float32(x.shape[-1]) + np.float32(eps))
        return O.round16(w * (x * r), dtype)

    assert _ulp_distance16(sum_not_mean(x, w), ref, dtype).max() > 1
    assert np.mean(weight_before_rounding(x, w) == ref) < 0.99
    # eps placement only shows on rows whose mean square is near eps
    xs = O.round16(np.full((1, 64), 1e-3, np.float32), dtype)
    assert _ulp_distance16(eps_outside(xs, w[:64]), _rmsnorm_f64(xs, w[:64], eps, dtype),
                           dtype).max() > 1
    assert _ulp_distance16(O.rmsnorm(xs, w[:64], eps, dtype),
                           _rmsnorm_f64(xs, w[:64], eps, dtype), dtype).max() <= 1


def test_rmsnorm_binary32_weight_promotes_and_unit_weight_normalises():
    rng = np.random.default_rng(3)
    x = O.round16(rng.standard_normal((3, 1000)).astype(np.float32), "f16")
    w32 = rng.uniform(0.5, 1.5, 1000).astype(np.float32)
    y = O.rmsnorm(x, w32, 1e-6, "f16", weight_f32=True)
    xn = O.rmsnorm(x, np.ones(1000, np.float32), 1e-6, "f16")
    np.testing.assert_array_equal(y, w32 * xn)            # no 16-bit rounding of the product
    np.testing.assert_allclose(np.mean(xn.astype(np.float64) ** 2, axis=-1), 1.0, rtol=2e-3)


def test_groupwise_weight_qdq_closed_forms():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((9, 300)) * 0.05).astype(np.float32)
    deq, q, s = O.groupwise_weight_qdq(w, group_size=1000)
    pdeq, pq, ps = O.per_output_weight_qdq(w)
    np.testing.assert_array_equal(q, pq)
    np.testing.assert_array_equal(s[:, 0], ps)
    np.testing.assert_array_equal(deq, pdeq)
    deq1, q1, s1 = O.groupwise_weight_qdq(w, group_size=1)
    assert s1.shape == (9, 300)
    # |w| >= 127 * 2**-14 keeps the scale unclamped: every such weight maps to
    # +-127; below it the scale clamps to 2**-14 and q = rint(w * 2**14).
    big = np.abs(w) >= 127 * 2.0 ** -14
    np.testing.assert_array_equal(np.abs(q1[big]), 127)
    np.testing.assert_array_equal(q1[~big], np.rint(w[~big].astype(np.float64) * 2 ** 14))
    np.testing.assert_array_equal(s1, O.scale_from_absmax(np.abs(w)))
    _, q128, s128 = O.groupwise_weight_qdq(w, group_size=128)       # 128 + 128 + 44
    assert s128.shape == (9, 3)
    np.testing.assert_array_equal(q128[:, 256:], O.per_output_weight_qdq(w[:, 256:])[1])


# --------------------------------------- torch-CPU restatement (cpu baseline)
def test_torch_path_equals_numpy_oracle():
    """oracle/torch_path.py (the timed CPU baseline) against the numpy oracle:
    scales, int8 values, int32 accumulators and binary32 outputs bit-equal on
    activations with x20 outlier channels, binary16 and binary32 inputs."""
    import torch

    from oracle import torch_path as T

    rng = np.random.default_rng(31)
    for m, n, k, dt in ((13, 90, 700, np.float16), (4, 33, 4096, np.float32),
                        (1, 16, 64, np.float16)):
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[:, rng.permutation(k)[:8]] *= 20
        x = x.astype(dt)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        _, qw, sw = O.per_output_weight_qdq(w)
        eout, eacc, exq, esx = O.w8a8_linear_dynamic(x, qw, sw, b, exact_int=True)
        xt = torch.from_numpy(x)
        sx = T.scale_from_absmax(xt.float().abs().amax(-1, keepdim=True))
        np.testing.assert_array_equal(sx.numpy(), esx)
        np.testing.assert_array_equal(T.quantize_symmetric(xt, sx).numpy(), exq)
        out, acc = T.per_token_linear(xt, torch.from_numpy(qw), torch.from_numpy(sw),
                                      torch.from_numpy(b))
        assert acc.dtype == torch.int32
        np.testing.assert_array_equal(acc.numpy(), eacc)
        np.testing.assert_array_equal(out.numpy(), eout)


def test_torch_path_tiny_kat_and_silu():
    import torch

    from oracle import torch_path as T

    kat = GOLDEN["tiny_int32_linear"]
    x = torch.tensor(kat["values"], dtype=torch.float32)
    w = np.array(kat["weight"], np.float32)
    _, qw, sw = O.per_output_weight_qdq(w)
    out, acc = T.per_token_linear(x, torch.from_numpy(qw), torch.from_numpy(sw),
                                  torch.tensor(kat["bias"], dtype=torch.float32))
    eout, eacc = O.integer_linear_per_output(
        x.numpy(), w, activation_scale=O.static_activation_scale(np.abs(x.numpy()).max()),
        bias=np.array(kat["bias"], np.float32))
    np.testing.assert_array_equal(acc.numpy(), eacc)
    np.testing.assert_array_equal(out.numpy(), eout)
    # SiLU*mul on an interleaved gate/up row: within one binary16 ulp of the
    # numpy restatement (both round SiLU(g) to binary16, then the product).
    g = np.random.default_rng(2).standard_normal((3, 64)).astype(np.float16) * 4
    gu = np.stack([g[:, :32], g[:, 32:]], axis=-1).reshape(3, 64)
    h = T.silu_mul(torch.from_numpy(gu)).numpy()
    eh = O.silu_mul_hf(g[:, :32], g[:, 32:])
    assert np.max(np.abs(h.astype(np.float32) - eh.astype(np.float32))
                  / np.maximum(np.abs(eh.astype(np.float32)), 2 ** -14)) <= 2 ** -10


def test_silu_mul_closed_form_matches_torch_silu_on_every_binary16():
    """The numpy closed form of SiLU*mul against torch's own CPU ``F.silu`` on
    binary16 tensors (the reference's ``act_fn(gate) * up``,
    lightweight_runner.py:358), which ``silu_mul_hf`` calls, over every finite
    binary16 gate, with up = 1 and with random up: at most one binary16 ulp
    apart, on a handful of values (3 of 63,488 observed; the two ``exp``
    implementations round a few inputs differently)."""
    import torch

    g = np.arange(65536, dtype=np.uint16).view(np.float16)
    g = g[np.isfinite(g)]
    rng = np.random.default_rng(20261202)
    for u in (np.ones_like(g), rng.standard_normal(g.shape).astype(np.float16)):
        with np.errstate(over="ignore"):
            got = O.silu_mul_closed_form(g, u)
        ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()

        def key(v):
            i = v.astype(np.float16).view(np.int16).astype(np.int32)
            return np.where(i < 0, -(i & 0x7FFF), i)
        d = np.abs(key(got) - key(ref))
        assert d.max() <= 1 and int((d > 0).sum()) <= 8
