"""Tolerance of the packed-F16 GEMM + epilogue checks (opcodes 1 / 16).

The GPU accumulates fp16 products in fp32 on MFMA; the oracle accumulates
exactly (double) and rounds once to fp16.  v is the GEMM value before the
epilogue (the oracle's fp16 readout), ref the oracle's output.

Where nothing cancels in the epilogue (|ref| >= |v| / 2: the bias or the
activation keeps at least half of v), the north star's 2e-3 relative bound
holds per element:

    |y - ref| <= 2e-3 * |ref| + 2^-24 + sqrt(K) * 2^-22 * sum_k |a_k w_k|

- 2e-3 * |ref|: the fp16 readout may land one fp16 ulp (at most 2^-10 |v|)
  away from the oracle's when the fp32 sum sits near a rounding boundary;
  with |ref| >= |v| / 2 that is at most 2^-9 |ref| = 1.95e-3 |ref| after a
  bias add, and the GELU / QuickGELU slope near the points where
  |ref| = |v| / 2 is below 1, so it stays inside there as well;
- 2^-24: the spacing of fp16 subnormals, the absolute resolution of the
  readout for |v| < 2^-14;
- the last term: fp32 accumulation error of a K-term dot product (random-walk
  growth sqrt(K) * unit roundoff, with a 4x margin), which matters only where
  the dot product itself cancels to near zero.

The reported relative figure (f16_max_rel) also leaves out elements whose
dot product cancels (the accumulation term above more than 1e-3 |ref|).

Where the epilogue cancels (|ref| < |v| / 2: a bias of opposite sign, or an
activation near zero), the error is relative to v, not to ref:

    |y - ref| <= 2e-3 * (|ref| + |v| + |bias|) + sqrt(K) * 2^-22 * sum_k |a_k w_k|
"""
import numpy as np


def f16_abs_dot(x, w_kn):
    """sum_k |fp16(x)_mk * w_kn| in double, [m][n]."""
    a = np.abs(x.astype(np.float16).astype(np.float64))
    return a @ np.abs(w_kn.astype(np.float64))


def no_cancellation(ref, v):
    """Elements whose epilogue keeps at least half of the GEMM value."""
    return np.abs(ref) >= 0.5 * np.abs(v)


def f16_bound(ref, v, bias_abs, absdot, k):
    accum = np.sqrt(k) * 2.0**-22 * absdot
    strict = 2e-3 * np.abs(ref) + 2.0**-24 + accum
    loose = 2e-3 * (np.abs(ref) + np.abs(v) + bias_abs) + accum
    return np.where(no_cancellation(ref, v), strict, loose)


def f16_max_rel(got, ref, v, absdot=None, k=None):
    """Largest |y - ref| / |ref| over the elements without cancellation whose
    |ref| is at least 2^-14 (outside the fp16 subnormal range): the figure
    the north star's 2e-3 relative bound speaks of.  Given absdot and k, the
    dot product's own cancellation is excluded too: elements whose fp32
    accumulation allowance (sqrt(K) * 2^-22 * sum_k |a_k w_k|) exceeds half of
    2e-3 |ref|, which long rows reach (K = 11520: about 4e-3 absolute)."""
    keep = no_cancellation(ref, v) & (np.abs(ref) >= 2.0**-14)
    if absdot is not None:
        keep &= np.sqrt(k) * 2.0**-22 * absdot <= 1e-3 * np.abs(ref)
    if not keep.any():
        return 0.0
    return float(np.max(np.abs(got[keep] - ref[keep]) / np.abs(ref[keep])))


def assert_f16_close(got, ref, v, bias_abs, absdot, k):
    bound = f16_bound(ref, v, bias_abs, absdot, k)
    assert np.all(np.isfinite(got))
    excess = np.abs(got - ref) - bound
    bad = excess > 0
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance; worst excess {float(excess.max()):.3g}"
    return f16_max_rel(got, ref, v, absdot, k)
