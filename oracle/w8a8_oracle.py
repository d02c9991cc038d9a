"""CPU oracle for the W8A8 quantized linear path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only to
check results against (or, for ``cpu_baseline``, as the timed CPU
restatement).  The product path under ``nano-pointllm_amd/`` never imports
it and never falls back to it.

Every function restates the reference algorithm it cites (paths relative to
the reference repository root).  Arithmetic follows the reference exactly:
IEEE binary32 division, ties-to-even rounding (``np.rint``), binary16
round-to-nearest-even for stored scales, exact integer accumulation, and a
dequant epilogue of separate binary32 roundings (``f32(acc) * s_x * s_w + b``).

How each function is pinned (tests/test_oracle.py):

* ``quantize_symmetric`` / ``scale_from_absmax`` - the reference's rounding and
  clipping KAT (tests/test_w8a8_contract.py:15-21), closed-form scale
  special cases (absmax 0, tiny, fp16 ties), brute force over all fp16 values
  against a float64 restatement.
* ``int32_matmul_*`` - two independent formulations (float64 BLAS, which is
  exact for |partial sums| < 2**53, and an int64 einsum) plus the reference
  package's integer golden fixture (tests/test_quantized_tensor_package.py:11-39)
  and the Dense64 caller-owned int8 fixture
  (architecture_simulator/tests/test_gtsu_cycle.py:443-465).
* ``integer_linear_per_output`` - the reference's tiny int32 linear KAT
  (tests/test_w8a8_contract.py:55-76) and the float64 "QDQ then FP" bound.
* ``dequant_epilogue`` - exact float64 recomputation of each rounding step.
* ``silu_mul_hf`` - computed with torch's own CPU ``F.silu`` (the reference's
  ``act_fn``); its numpy closed form ``silu_mul_closed_form`` is within one
  binary16 ulp of float64, and the two differ on 3 of the 63,488 finite
  binary16 gates, by one ulp.
* ``requantize_int32`` / ``compile_requant_ratio`` - the 12 locked vectors of
  architecture_simulator/gtsu_cycle/requant.py:122-136 and their asserted
  outputs (architecture_simulator/tests/test_gtsu_cycle.py:666-675).
* ``dequantize_int32_to_bf16`` - the 12 locked vectors of
  architecture_simulator/gtsu_cycle/bf16_dequant.py:80-94 with their asserted
  outputs, and 1000 random vectors against float64 -> bf16 RNE
  (architecture_simulator/tests/test_gtsu_cycle.py:690-721).
* ``pack_gateup_rows`` / ``pack_qkv_rows`` - packed == unpacked invariants
  (tests/test_lightweight_runner.py:132-200).
* ``groupwise_weight_qdq`` - two closed forms: a group of at least K columns
  is ``per_output_weight_qdq``; a group of one column maps every weight with
  |w| >= 127 * 2**-14 to +-127 and every smaller one to rint(w * 2**14).
* ``residual_add`` / ``smooth_divide`` - numpy's and torch's own 16-bit
  arithmetic (convert to binary32, operate, round once) on random and
  boundary values.
* ``rmsnorm`` - a float64 restatement within one 16-bit ulp; bit equality on
  inputs whose binary32 sum of squares is exact in any order; planted
  mistakes (eps outside the square root, sum instead of mean, weight before
  the rounding) fail.  The binary32 summation order of torch's CPU ``mean``
  is not pinned: GPU parity for the normalization is by tolerance, and the
  quantization of the GPU's own normalized rows is bit-exact.
"""
from __future__ import annotations

import math
import struct

import numpy as np

SYMMETRIC_MIN = -127
SYMMETRIC_MAX = 127
# torch.finfo(torch.float16).tiny == 2**-14 (nanopointllm/compression/w8a8.py:48)
SCALE_MIN = np.float32(2.0 ** -14)
INT32_MIN = -(1 << 31)
INT32_MAX = (1 << 31) - 1


# --------------------------------------------------------------------------
# a2 / a3 / a4 / a5 / a6: scales and quantization
# --------------------------------------------------------------------------
def scale_from_absmax(absmax) -> np.ndarray:
    """``nanopointllm/compression/w8a8.py:46-50``.

    ``s = max(f32(f16_rne(max(absmax, 2**-14) / 127)), 2**-14)`` with the
    division in binary32.
    """
    a = np.asarray(absmax, dtype=np.float32)
    raw = np.maximum(a, SCALE_MIN) / np.float32(SYMMETRIC_MAX)
    return np.maximum(raw.astype(np.float16).astype(np.float32), SCALE_MIN)


def quantize_symmetric(values, scale) -> np.ndarray:
    """``nanopointllm/compression/w8a8.py:33-43``.

    ``q = clamp(rne(f32(x) / f32(s)), -127, 127)`` as int8.  Non-positive
    scales raise ``ValueError("quantization scale must be positive")``.
    """
    s = np.asarray(scale, dtype=np.float32)
    if np.any(s <= 0):
        raise ValueError("quantization scale must be positive")
    v = np.asarray(values).astype(np.float32)
    q = np.rint(v / s)
    return np.clip(q, SYMMETRIC_MIN, SYMMETRIC_MAX).astype(np.int8)


def groupwise_weight_qdq(weight, group_size: int = 128):
    """``groupwise_weight_qdq`` (nanopointllm/compression/w8a8.py:65-91): one
    scale per row and group of ``group_size`` columns (the last group may be
    shorter).  Returns (dequant f32, int8, scales f32 [rows, groups])."""
    w = np.asarray(weight, dtype=np.float32)
    rows = w.shape[0]
    flat = w.reshape(rows, -1)
    cols = flat.shape[1]
    groups = (cols + group_size - 1) // group_size
    q = np.empty(flat.shape, np.int8)
    deq = np.empty(flat.shape, np.float32)
    scales = np.empty((rows, groups), np.float32)
    for g in range(groups):
        part = flat[:, g * group_size: min(cols, (g + 1) * group_size)]
        s = scale_from_absmax(np.abs(part).max(axis=1))
        q[:, g * group_size: g * group_size + part.shape[1]] = quantize_symmetric(part, s[:, None])
        deq[:, g * group_size: g * group_size + part.shape[1]] = (
            q[:, g * group_size: g * group_size + part.shape[1]].astype(np.float32) * s[:, None])
        scales[:, g] = s
    return deq.reshape(w.shape), q.reshape(w.shape), scales


def static_activation_scale(absmax) -> np.ndarray:
    """``nanopointllm/compression/w8a8.py:94-98`` (one tensor-wide absmax)."""
    value = np.asarray(absmax, dtype=np.float32)
    if value.size != 1:
        raise ValueError("static activation scale expects one tensor-wide absmax")
    return scale_from_absmax(value.reshape(()))


def row_absmax(values) -> np.ndarray:
    """``|x|.amax(dim=-1, keepdim=True)`` in binary32 (w8a8.py:112)."""
    v = np.asarray(values).astype(np.float32)
    return np.abs(v).max(axis=-1, keepdims=True)


def dynamic_per_token_quant(values) -> tuple[np.ndarray, np.ndarray]:
    """Integer half of ``dynamic_per_token_activation_qdq`` (w8a8.py:106-115).

    Returns ``(q int8 [..., K], scales f32 [..., 1])``.
    """
    scales = scale_from_absmax(row_absmax(values))
    return quantize_symmetric(values, scales), scales


def dynamic_per_token_activation_qdq(values) -> tuple[np.ndarray, np.ndarray]:
    """``nanopointllm/compression/w8a8.py:106-115`` (QDQ values in x's dtype)."""
    v = np.asarray(values)
    q, scales = dynamic_per_token_quant(v)
    return (q.astype(np.float32) * scales).astype(v.dtype), scales


def per_output_weight_qdq(weight) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``nanopointllm/compression/w8a8.py:53-62``.

    Per output row: absmax -> ``scale_from_absmax`` -> ``quantize_symmetric``.
    Returns ``(dequantized in weight dtype, int8 [N, K], f32 scales [N])``.
    """
    w = np.asarray(weight)
    if w.ndim < 2:
        raise ValueError("weight must have at least two dimensions")
    rows = w.astype(np.float32).reshape(w.shape[0], -1)
    scales = scale_from_absmax(np.abs(rows).max(axis=1))
    q = quantize_symmetric(rows, scales[:, None])
    deq = (q.astype(np.float32) * scales[:, None]).reshape(w.shape)
    return deq.astype(w.dtype), q.reshape(w.shape), scales


# --------------------------------------------------------------------------
# a8: int8 x int8 -> int32 and the dequant epilogue
# --------------------------------------------------------------------------
def int32_matmul_f64(a_i8, w_i8) -> np.ndarray:
    """Exact ``int32(a) @ int32(w).T`` through float64 BLAS.

    Every product and partial sum is an integer of magnitude below
    ``K * 127**2 < 2**31 < 2**53`` so float64 accumulation is exact in any
    order.
    """
    a = np.asarray(a_i8)
    w = np.asarray(w_i8)
    if a.shape[-1] * SYMMETRIC_MAX * SYMMETRIC_MAX >= (1 << 31):
        raise OverflowError("worst-case dot product exceeds signed INT32")
    out = a.astype(np.float64) @ w.astype(np.float64).T
    return out.astype(np.int32)


def int32_matmul_int(a_i8, w_i8) -> np.ndarray:
    """``int32(a) @ int32(w).T`` with numpy integer arithmetic.

    This is the literal restatement of the reference's CPU
    ``flat @ qweight_cpu.transpose(0, 1)`` (w8a8.py:131-133); the
    ``cpu_baseline`` times this form.
    """
    a = np.asarray(a_i8).astype(np.int32)
    w = np.asarray(w_i8).astype(np.int32)
    return a @ w.T


def dequant_epilogue(acc, sx, sw, bias=None) -> np.ndarray:
    """``nanopointllm/compression/w8a8.py:134-137``.

    ``out = f32(acc); out *= s_x; out *= s_w[None, :]; out += bias[None, :]``,
    each step rounded to binary32 (no fused multiply-add).
    """
    out = np.asarray(acc).astype(np.float32)
    out = out * np.asarray(sx, dtype=np.float32)
    out = out * np.asarray(sw, dtype=np.float32)[None, :]
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float32)[None, :]
    return out.astype(np.float32)


def integer_linear_per_output(values, weight, *, activation_scale, bias=None):
    """``integer_linear_per_output_reference`` (w8a8.py:118-139).

    Returns ``(out f32 [..., N], acc int32 [..., N])``.
    """
    v = np.asarray(values)
    w = np.asarray(weight)
    if w.ndim != 2 or v.shape[-1] != w.shape[1]:
        raise ValueError("linear input/weight shapes do not match")
    qa = quantize_symmetric(v, activation_scale)
    _, qw, sw = per_output_weight_qdq(w)
    flat = qa.reshape(-1, qa.shape[-1])
    acc = int32_matmul_f64(flat, qw)
    out = dequant_epilogue(acc, np.asarray(activation_scale, np.float32), sw, bias)
    return (out.reshape(*v.shape[:-1], w.shape[0]),
            acc.reshape(*v.shape[:-1], w.shape[0]))


def linear_from_quantized(xq, sx, wq, sw, bias=None, *, exact_int=False):
    """Per-token W8A8 linear on already-quantized operands.

    ``acc = xq @ wq.T`` then :func:`dequant_epilogue`; returns
    ``(out f32 [M, N], acc int32 [M, N])``.
    """
    acc = int32_matmul_int(xq, wq) if exact_int else int32_matmul_f64(xq, wq)
    return dequant_epilogue(acc, np.asarray(sx, np.float32).reshape(-1, 1), sw, bias), acc


def w8a8_linear_dynamic(x, wq, sw, bias=None, *, exact_int=False):
    """Per-token dynamic A8 x per-output W8 linear (the runtime contract).

    ``x`` is the [M, K] activation (fp16/bf16/f32 values), ``wq``/``sw`` the
    per-output int8 weight and scales.  Returns ``(out f32, acc int32,
    xq int8, sx f32 [M, 1])``.
    """
    xq, sx = dynamic_per_token_quant(x)
    out, acc = linear_from_quantized(xq, sx, wq, sw, bias, exact_int=exact_int)
    return out, acc, xq, sx


# --------------------------------------------------------------------------
# a12 / a14 / a15: packing and SiLU*mul
# --------------------------------------------------------------------------
def pack_qkv_rows(wq, wk, wv) -> np.ndarray:
    """``torch.cat([Wq, Wk, Wv], dim=0)`` (llama/paged_attention.py:1242-1245)."""
    return np.concatenate([wq, wk, wv], axis=0)


def pack_gateup_rows(wg, wu, layout: str) -> np.ndarray:
    """``_pack_gateup_tensors`` (llama/lightweight_runner.py:57-93)."""
    if layout == "split":
        return np.concatenate([wg, wu], axis=0)
    if layout == "interleave":
        return np.stack([wg, wu], axis=1).reshape(wg.shape[0] * 2, *wg.shape[1:])
    raise ValueError(f"unsupported gate_up weight layout: {layout}")


def silu_mul_hf(g16, u16) -> np.ndarray:
    """``act_fn(gate) * up`` on binary16 tensors (lightweight_runner.py:358),
    with the reference's own ``act_fn``: torch's CPU ``F.silu`` (SiLU in
    binary32 rounded to binary16), then the binary16 product (exact in
    binary32, one rounding to binary16)."""
    import torch

    g = torch.from_numpy(np.ascontiguousarray(g16, dtype=np.float16))
    u = torch.from_numpy(np.ascontiguousarray(u16, dtype=np.float16))
    return (torch.nn.functional.silu(g) * u).numpy()


def silu_mul_closed_form(g16, u16) -> np.ndarray:
    """``silu_mul_hf`` restated in numpy: SiLU in binary32 ``g / (1 + exp(-g))``
    rounded to binary16, then the binary16 product.  numpy's and torch's
    binary32 ``exp`` round a few inputs differently (see the header)."""
    g = np.asarray(g16, dtype=np.float16).astype(np.float32)
    u = np.asarray(u16, dtype=np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        s = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float16)
    return (s.astype(np.float32) * u).astype(np.float16)


def gateup_silu_mul_from_acc(acc, sx, sgu, bias=None, *, layout="interleave"):
    """Packed gate/up epilogue: dequant -> binary16 -> SiLU(g) * u.

    ``acc`` is the int32 [M, 2*I] accumulator of the packed projection in the
    given row layout.  Returns the binary16 [M, I] product.
    """
    y16 = dequant_epilogue(acc, np.asarray(sx, np.float32).reshape(-1, 1), sgu, bias).astype(np.float16)
    inter = y16.shape[1] // 2
    if layout == "interleave":
        g, u = y16[:, 0::2], y16[:, 1::2]
    else:
        g, u = y16[:, :inter], y16[:, inter:]
    return silu_mul_hf(g, u)


# --------------------------------------------------------------------------
# a17: INT32 -> A8 requant (multiplier / right shift)
# --------------------------------------------------------------------------
def _fp16(value: float) -> float:
    return struct.unpack("e", struct.pack("e", value))[0]


def compile_requant_ratio(ratio: float) -> tuple[int, int]:
    """``architecture_simulator/gtsu_cycle/requant.py:80-95``."""
    if ratio <= 0 or not math.isfinite(ratio):
        raise ValueError("requant ratio must be positive and finite")
    max_mult = (1 << 32) - 1
    shift = min(63, math.floor(math.log2(max_mult / ratio)))
    if shift < 0:
        raise OverflowError("requant ratio exceeds UINT32 multiplier range")
    mult = round(ratio * (1 << shift))
    if mult > max_mult:
        shift -= 1
        mult = round(ratio * (1 << shift))
    if mult <= 0 or shift < 0:
        raise OverflowError("requant ratio is outside multiplier/shift range")
    return mult, shift


def compile_fp16_requant_scale(activation_scale, weight_scale, output_scale):
    """``architecture_simulator/gtsu_cycle/requant.py:62-77``.

    Returns ``(multiplier, right_shift, exact_ratio, relative_error)``.
    """
    a, w, o = _fp16(activation_scale), _fp16(weight_scale), _fp16(output_scale)
    if min(a, w, o) <= 0 or not all(math.isfinite(t) for t in (a, w, o)):
        raise ValueError("requant scales must be positive finite FP16 values")
    ratio = a * w / o
    mult, shift = compile_requant_ratio(ratio)
    represented = mult / (1 << shift)
    return mult, shift, ratio, abs(represented - ratio) / ratio


def requantize_int32(acc: int, bias: int, multiplier: int, right_shift: int) -> int:
    """``architecture_simulator/gtsu_cycle/requant.py:98-119``.

    ``(acc + bias) * multiplier``, ties-to-even on the magnitude at the right
    shift, sign restored, clipped to [-127, 127].
    """
    if not INT32_MIN <= acc <= INT32_MAX:
        raise ValueError("accumulator exceeds INT32")
    if not INT32_MIN <= bias <= INT32_MAX:
        raise ValueError("bias exceeds INT32")
    if not 0 <= multiplier < (1 << 32):
        raise ValueError("multiplier exceeds UINT32")
    if not 0 <= right_shift <= 63:
        raise ValueError("right_shift must be in [0, 63]")
    product = (acc + bias) * multiplier
    mag = abs(product)
    if right_shift:
        t = mag >> right_shift
        rem = mag & ((1 << right_shift) - 1)
        half = 1 << (right_shift - 1)
        if rem > half or (rem == half and (t & 1)):
            t += 1
    else:
        t = mag
    r = -t if product < 0 else t
    return max(SYMMETRIC_MIN, min(SYMMETRIC_MAX, r))


# --------------------------------------------------------------------------
# a18: INT32 x FP16 x FP16 -> BF16 with one rounding
# --------------------------------------------------------------------------
def _decode_fp16_bits(bits: int) -> tuple[int, int, int]:
    if not 0 <= bits < (1 << 16):
        raise ValueError("FP16 scale bits exceed 16 bits")
    sign = bits >> 15
    exponent = (bits >> 10) & 0x1F
    fraction = bits & 0x3FF
    if exponent == 0x1F:
        raise ValueError("BF16 dequant scales must be finite FP16 values")
    if exponent == 0:
        return fraction, -24, sign
    return 1024 + fraction, exponent - 25, sign


def _rne_shift(value: int, shift: int) -> int:
    if shift <= 0:
        return value << -shift
    t = value >> shift
    rem = value & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    return t + int(rem > half or (rem == half and (t & 1)))


def dequantize_int32_to_bf16(acc: int, sa_bits: int, sw_bits: int) -> int:
    """``architecture_simulator/gtsu_cycle/bf16_dequant.py:47-77``.

    Exact product ``acc * s_a * s_w`` rounded once to bf16 (RNE, subnormals
    kept, overflow to inf).  Returns the bf16 bit pattern.
    """
    if not INT32_MIN <= acc <= INT32_MAX:
        raise ValueError("accumulator exceeds INT32")
    ma, ea, sa = _decode_fp16_bits(sa_bits)
    mw, ew, sw = _decode_fp16_bits(sw_bits)
    if acc == 0 or ma == 0 or mw == 0:
        return 0
    sign = int(acc < 0) ^ sa ^ sw
    product = abs(acc) * ma * mw
    exponent = ea + ew
    top = product.bit_length() - 1
    unbiased = top + exponent
    if unbiased < -126:
        frac = _rne_shift(product, -(exponent + 133))
        if frac == 0:
            return sign << 15
        if frac >= 128:
            return (sign << 15) | (1 << 7)
        return (sign << 15) | frac
    sig = _rne_shift(product, top - 7)
    if sig >= 256:
        sig >>= 1
        unbiased += 1
    if unbiased > 127:
        return (sign << 15) | 0x7F80
    return (sign << 15) | ((unbiased + 127) << 7) | (sig - 128)


# --------------------------------------------------------------------------
# activation prologue: residual add, RMSNorm, SmoothQuant divide
# --------------------------------------------------------------------------
def round16(values, dtype: str) -> np.ndarray:
    """Round binary32 values to ``"f16"`` / ``"bf16"`` (RNE) and back."""
    v = np.asarray(values, dtype=np.float32)
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(v)).reshape(v.shape)
    raise ValueError(f"unsupported 16-bit dtype: {dtype}")


def residual_add(hidden, residual, dtype: str) -> np.ndarray:
    """``summed = hidden_states + residual`` on 16-bit tensors
    (``LightweightRMSNorm.residual_norm``, llama/lightweight_runner.py:256)."""
    return round16(np.asarray(hidden, np.float32) + np.asarray(residual, np.float32), dtype)


def rmsnorm(hidden, weight, eps: float, dtype: str, *, weight_f32: bool = False) -> np.ndarray:
    """``LightweightRMSNorm.forward`` (llama/lightweight_runner.py:239-245).

    ``x = f32(h); x = x * rsqrt(mean(x**2) + eps); y = weight * x.to(dtype)``.
    A 16-bit weight rounds ``y`` to ``dtype``; a binary32 weight promotes it
    to binary32 (torch's type promotion).
    """
    x = np.asarray(hidden, np.float32)
    var = np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32) / np.float32(x.shape[-1])
    r = np.float32(1.0) / np.sqrt(var + np.float32(eps))
    xn = round16(x * r, dtype)
    y = np.asarray(weight, np.float32) * xn
    return y.astype(np.float32) if weight_f32 else round16(y, dtype)


def smooth_divide(values, smoothing, dtype: str | None) -> np.ndarray:
    """``values / smoothing.to(values.dtype)`` of the SmoothQuant input hook
    (compression/w8a8.py:351-359); ``dtype`` None keeps binary32 values."""
    out = np.asarray(values, np.float32) / np.asarray(smoothing, np.float32)
    return out.astype(np.float32) if dtype is None else round16(out, dtype)


# --------------------------------------------------------------------------
# bfloat16 helpers (numpy has no bf16 dtype)
# --------------------------------------------------------------------------
def f32_to_bf16_bits(values) -> np.ndarray:
    """Round binary32 to bfloat16 (ties to even); returns uint16 bit patterns."""
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = v.view(np.uint32).astype(np.uint64)
    rounding = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    out = ((u + rounding) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(v)
    if np.any(nan):
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


# --------------------------------------------------------------------------
# a9: error metrics
# --------------------------------------------------------------------------
def tensor_error(reference, candidate) -> dict[str, float]:
    """``_tensor_error`` (nanopointllm/compression/w8a8.py:254-262)."""
    ref = np.asarray(reference, dtype=np.float32)
    diff = np.asarray(candidate, dtype=np.float32) - ref
    denom = np.maximum(np.abs(ref), np.float32(1e-8))
    return {
        "rmse": float(np.sqrt(np.mean(np.square(diff)))),
        "max_abs": float(np.max(np.abs(diff))),
        "mean_abs": float(np.mean(np.abs(diff))),
        "mean_relative_abs": float(np.mean(np.abs(diff) / denom)),
    }
