"""Tolerance of the packed-F16 GEMM + epilogue checks (opcodes 1 / 16).

The GPU accumulates fp16 products in fp32 on MFMA; the oracle accumulates
exactly (double) and rounds once to fp16.  Per element:

    |y - ref| <= 2e-3 * (|ref| + |v| + |bias|) + sqrt(K) * 2^-22 * sum_k |a_k w_k|

- 2e-3 relative: one fp16 ulp of v (2^-10 |v|) from the fp16 readout landing
  on the other side of a rounding boundary, carried through the bias add and
  the 1.13-Lipschitz GELU / QuickGELU;
- the second term: fp32 accumulation error of a K-term dot product (random-walk
  growth sqrt(K) * unit roundoff, with a 4x margin), which matters only where
  the sum cancels to near zero.
"""
import numpy as np


def f16_abs_dot(x, w_kn):
    """sum_k |fp16(x)_mk * w_kn| in double, [m][n]."""
    a = np.abs(x.astype(np.float16).astype(np.float64))
    return a @ np.abs(w_kn.astype(np.float64))


def f16_bound(ref, v, bias_abs, absdot, k):
    return 2e-3 * (np.abs(ref) + np.abs(v) + bias_abs) + np.sqrt(k) * 2.0**-22 * absdot


def assert_f16_close(got, ref, v, bias_abs, absdot, k):
    bound = f16_bound(ref, v, bias_abs, absdot, k)
    assert np.all(np.isfinite(got))
    excess = np.abs(got - ref) - bound
    bad = excess > 0
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance; worst excess {float(excess.max()):.3g}"
