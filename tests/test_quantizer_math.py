"""The fast dynamic-scale quantizer of the fused decode kernel, restated on the
host with the same IEEE operations the kernel runs, and checked against the
exact answer.

quant8_dyn (csrc/w8a8_common.h) computes t = fma(x, r, 1.5 * 2^23) with
r = fl32(1/s): 1.5 * 2^23 plus the integer nearest the exact product x * r,
whose low byte is the int8 result.  It keeps that value unless the exact
remainder e = fma(x, r, -(t - 1.5 * 2^23)) has |e| >= 0.5 - 2^-14 (x * r
near a half-integer), where the wavefront redoes the chunk with the exact tie
test.  The fused multiply-adds are restated in float64: x * r has at most
11 + 24 significant bits, so float64 holds the product exactly and the sums
within 2^-29, after which one rounding to binary32 follows.  That 2^-29 can
move the binary32 rounding only within 2^-29 of a half-integer, inside the
band the fallback takes, so the restated fast path is the hardware's.
The claim pinned here: whenever the fast path is taken, it equals the
correctly rounded (ties to even) quotient of quantize_symmetric
(nanopointllm/compression/w8a8.py:33-43), for every finite binary16 and
bfloat16 x in the dynamic range |x| <= 127.07 s and binary16 scales across
the whole range.  The exact quotient is rint(float64(x) / float64(s)): x / s
is either a half-integer (exact in float64) or at least 2^-12 from one, far
beyond float64's rounding error at |x / s| < 128.
"""
from __future__ import annotations

import numpy as np
import pytest

THRESH = np.float32(0.5 - 2.0 ** -14)
MAGIC = 1.5 * 2.0 ** 23


def _all_finite(kind: str) -> np.ndarray:
    bits = np.arange(65536, dtype=np.uint32)
    if kind == "f16":
        x = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    else:
        x = (bits << 16).view(np.float32)
    return x[np.isfinite(x)]


def _scales() -> np.ndarray:
    rng = np.random.default_rng(5)
    a = np.ldexp(1.0 + rng.integers(0, 1024, 400) / 1024.0, rng.integers(-20, 20, 400))
    s = (a / 127.0).astype(np.float16).astype(np.float32)
    s = np.maximum(s, np.float32(2.0 ** -14))
    extra = np.float32([2.0 ** -14, 1.0, 0.25, np.float16(1.0 / 127)])
    return np.unique(np.concatenate([s[np.isfinite(s)], extra]))


def _fast_path(x: np.ndarray, s: np.float32):
    """(value, taken) of the fast path, and the int8 read from t's low byte."""
    r = np.float32(1.0) / s
    p = x.astype(np.float64) * np.float64(r)                # exact
    t = (p + MAGIC).astype(np.float32)                     # fma(x, r, MAGIC)
    n = t.astype(np.float64) - MAGIC                       # exact
    e = (p - n).astype(np.float32)                         # fma(x, r, MAGIC - t)
    low = (t.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
    np.testing.assert_array_equal(low.astype(np.float64), n)
    return n.astype(np.float32), np.abs(e) < THRESH


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_fast_path_is_exact_for_dynamic_scales(kind):
    x_all = _all_finite(kind)
    fast_total = slow_total = 0
    for s in _scales():
        x = x_all[np.abs(x_all) <= np.float32(127.0625) * s]
        t, fast = _fast_path(x, s)
        exact = np.rint(x.astype(np.float64) / np.float64(s))
        np.testing.assert_array_equal(t[fast], exact[fast].astype(np.float32),
                                      err_msg=f"{kind} scale {s}")
        assert np.abs(t).max() <= 127
        fast_total += int(fast.sum())
        slow_total += int((~fast).sum())
    # the vote is rare: the exact fallback is taken for well under 1% of values
    assert slow_total < 0.01 * (fast_total + slow_total)


def test_fast_path_flags_every_tie():
    """Exact ties (x / s = k + 1/2) always fall back, and wherever the nearest
    integer to x * r is not the correctly rounded x / s, the fallback is taken."""
    s = np.float32(2.0)
    x = np.arange(-254, 255, dtype=np.float32)          # x / s hits every half-integer
    t, fast = _fast_path(x, s)
    ties = (x % 2) != 0
    assert not fast[ties].any()
    # An inexact r can put x * r on the other side of a half-integer than
    # x / s.  Find scales where that happens and check the fallback takes them.
    found = False
    xs = _all_finite("f16")
    for sc in _scales():
        x = xs[np.abs(xs) <= np.float32(127.0625) * sc]
        t, fast = _fast_path(x, sc)
        exact = np.rint(x.astype(np.float64) / np.float64(sc))
        wrong = t != exact
        if wrong.any():
            found = True
            assert not fast[wrong].any()
    assert found, "no scale where plain rint(x * r) is wrong: the fallback would be untested"
