"""Shared helpers for the parity tests (fp16 bit handling, tolerance checks)."""
from __future__ import annotations

import numpy as np


def f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def f32(bits):
    return f16(bits).astype(np.float32)


def close_report(actual_bits, expected, atol, rtol):
    """|a - e| <= atol + rtol*|e| elementwise (test_utils.hpp:30-62).  `expected`
    is fp16 bits (uint16) or float32 exact values.  Returns (ok, max_abs, n_bad)."""
    a = f32(actual_bits).astype(np.float64)
    if expected.dtype == np.uint16:
        e = f32(expected).astype(np.float64)
    else:
        e = np.asarray(expected, dtype=np.float64)
    diff = np.abs(a - e)
    bad = ~(diff <= atol + rtol * np.abs(e))
    return (not bad.any()) and np.isfinite(a).all(), float(diff.max(initial=0.0)), int(bad.sum())


def assert_close(actual_bits, expected, atol, rtol, what=""):
    ok, mx, nbad = close_report(actual_bits, expected, atol, rtol)
    assert ok, f"{what}: {nbad} elements outside atol={atol} rtol={rtol}; max |diff| = {mx:.3e}"


def ulp_diff(a_bits, b_bits):
    """Distance in fp16 ulps between two arrays of finite fp16 bit patterns."""
    def ordered(x):
        x = np.asarray(x, dtype=np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x & 0x7FFF)
    return np.abs(ordered(a_bits) - ordered(b_bits))
