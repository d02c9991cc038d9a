"""The fast dynamic-scale quantizer of the fused decode kernel, restated on the
host with binary32 numpy arithmetic (the same IEEE operations the kernel
runs) and checked against the exact answer.

quant8_dyn (csrc/w8a8_common.h) takes rint(x * r), r = fl32(1/s), as the
quantized value of x / s unless fl32(x * r) lies within 2^-15 of a
half-integer, where the wavefront redoes the chunk with the exact tie test.
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

THRESH = np.float32(0.5 - 2.0 ** -15)


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
    r = np.float32(1.0) / s
    y = x * r
    t = np.rint(y)
    return t, np.abs(y - t) < THRESH


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
    """Exact ties (x / s = k + 1/2) always fall back, and a planted wider
    threshold (ignoring the 2^-15 margin) would accept a wrong rounding."""
    s = np.float32(2.0)
    x = np.arange(-254, 255, dtype=np.float32)          # x / s hits every half-integer
    t, fast = _fast_path(x, s)
    ties = (x % 2) != 0
    assert not fast[ties].any()
    # With a threshold of exactly 0.5 a tie would pass as a fast value whose
    # rint rounds to even; a near-tie from an inexact r would not.  Find a scale
    # where fl32(x * r) lands on the wrong side of a half-integer.
    found = False
    xs = _all_finite("f16")
    for sc in _scales():
        x = xs[np.abs(xs) <= np.float32(127.0625) * sc]
        y = x * (np.float32(1.0) / sc)
        exact = np.rint(x.astype(np.float64) / np.float64(sc))
        wrong = np.rint(y) != exact
        if wrong.any():
            found = True
            assert (np.abs(y - np.rint(y))[wrong] >= THRESH).all()
    assert found, "no scale where plain rint(x * r) is wrong: the fallback would be untested"
