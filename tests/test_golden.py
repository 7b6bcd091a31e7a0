"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the C oracle).

CPU tests re-derive every fixture from closed forms that do not go through
the oracle -- the reference's blob and permuted-F16 address formulas
(op_executor.cc:321-335 + linear_w8a8.c:453,482,486-488; test.c:547-558),
an int64 brute-force product, per-operation float32 numpy restatements of
linear_w8a8.c:34-59 and :159-179, and float64 F16 products with the
mat_mul.c:788-826 activations -- and check that the oracle still reproduces
them bit for bit.  GPU tests run the HIP path on the same inputs through the
C ABI: W8A8 bit-exact, F16 within the tolerance of tests/tolerances.py.
"""
import os

import numpy as np
import pytest

from tolerances import assert_f16_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_cases(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as data:
        cases = {}
        for key in data.files:
            case, field = key.split("/")
            cases.setdefault(case, {})[field] = data[key]
    return cases


W8A8 = load_cases("w8a8_golden.npz")
F16 = load_cases("f16_golden.npz")


def dims(case, *names):
    return tuple(int(case[n]) for n in names)


# ---- independent restatements ---------------------------------------------------

def blob_weights(blob, k, n):
    """W(n,k) read with the reference's deep-tile address formula."""
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    off = (128 + (nn // 64) * 64 * k + (kk // 32) * 2048 + ((nn % 64) // 32) * 1024 + ((kk % 32) // 4) * 128 +
           (nn % 32) * 4 + kk % 4)
    return blob[off].view(np.int8)


def blob_columns(blob, k, n):
    base = 128 + k * n
    sw = blob[base:base + 4 * n].view(np.float32)
    sums = blob[base + 4 * n:base + 8 * n].view(np.int32)
    inv = blob[base + 8 * n:base + 8 * n + 4 * k].view(np.float32)
    return sw, sums, inv


def numpy_quantize(x, inv):
    f = np.float32
    t = (x * inv[None, :]).astype(f)
    a = np.abs(t).max(axis=1)
    s = np.maximum((a / f(127.0)).astype(f), f(1e-12))
    r = (f(1.0) / s).astype(f)
    v = ((t * r[:, None]).astype(f) + f(128.0)).astype(f)
    bits = np.clip(v.view(np.int32), np.float32(1.0).view(np.int32), np.float32(255.0).view(np.int32))
    return np.rint(bits.view(np.float32)).astype(np.uint8), s


def numpy_output(acc, sums, sw, s):
    c = (acc.astype(np.int64) - (sums.astype(np.int64) << 7)).astype(np.int64)
    c = ((c + 2**31) % 2**32 - 2**31).astype(np.int32)
    return ((c.astype(np.float32) * sw[None, :]).astype(np.float32) * s[:, None]).astype(np.float32)


def permuted_f16(w, k, n):
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    idx = ((nn // 32) * (k // 32) + kk // 32) * 1024 + ((kk % 32) // 2) * 64 + (nn % 32) * 2 + kk % 2
    return w[idx].view(np.float16)  # [k][n]


def f16_reference(case):
    m, k, n, channels, mode = dims(case, "m", "k", "n", "channels", "mode")
    a = case["x"].astype(np.float16).astype(np.float64)
    wk = permuted_f16(case["w"], k, n).astype(np.float64)
    v = (a @ wk).astype(np.float16).astype(np.float32)
    bias = case.get("bias")
    if mode == 3:
        z = v[:, :channels].T.astype(np.float64)
        if bias is not None:
            z = z + bias[:, None]
        return z, v[:, :channels].T, wk
    z = v.astype(np.float64) + (bias[None, :] if bias is not None else 0.0)
    if mode == 1:
        z = z / (1.0 + np.exp(-1.5957691216057308 * (z + 0.044715 * z * z * z)))
    elif mode == 2:
        z = z / (1.0 + np.exp(-1.702 * z))
    return z, v, wk


# ---- CPU ------------------------------------------------------------------------

@pytest.mark.parametrize("name", sorted(W8A8))
def test_w8a8_fixture_matches_closed_forms(name):
    case = W8A8[name]
    m, k, n = dims(case, "m", "k", "n")
    sw, sums, inv = blob_columns(case["blob"], k, n)
    u, s = numpy_quantize(case["x"], inv)
    np.testing.assert_array_equal(u, case["u"])
    np.testing.assert_array_equal(s.view(np.uint32), case["s"].view(np.uint32))
    acc = case["u"].astype(np.int64) @ blob_weights(case["blob"], k, n).T.astype(np.int64)
    np.testing.assert_array_equal(acc, case["acc"].astype(np.int64))
    y = numpy_output(case["acc"], sums, sw, case["s"])
    np.testing.assert_array_equal(y.view(np.uint32), case["y"].view(np.uint32))


def test_w8a8_special_rows_fixture():
    case = W8A8["special_rows"]
    assert case["s"][0] == np.float32(1e-12) and np.all(case["u"][0] == 128)
    assert case["s"][1] == np.float32(1.0)
    assert list(case["u"][1, :5]) == [128, 130, 130, 128, 255]
    assert np.all(case["u"][2] == 128)


@pytest.mark.parametrize("name", sorted(W8A8))
def test_oracle_reproduces_w8a8_fixture(orc, name):
    case = W8A8[name]
    m, k, n = dims(case, "m", "k", "n")
    assert orc.check_header(case["blob"], k, n) == 0
    _, _, inv = blob_columns(case["blob"], k, n)
    u, s = orc.quantize(case["x"], inv)
    np.testing.assert_array_equal(u, case["u"])
    np.testing.assert_array_equal(orc.accumulate(u, case["blob"], k, n), case["acc"])
    y = orc.linear(case["x"], case["blob"], k, n)
    np.testing.assert_array_equal(y.view(np.uint32), case["y"].view(np.uint32))


@pytest.mark.parametrize("name", sorted(F16))
def test_f16_fixture_matches_float64(name):
    case = F16[name]
    z, _, _ = f16_reference(case)
    assert np.all(np.abs(case["y"] - z) <= 2e-3 * np.abs(z) + 1e-6)


@pytest.mark.parametrize("name", sorted(F16))
def test_oracle_reproduces_f16_fixture(orc, name):
    case = F16[name]
    m, k, n, channels, mode = dims(case, "m", "k", "n", "channels", "mode")
    y = orc.f16_gemm_epilogue(case["x"], case["w"], case.get("bias"), m, k, n, channels, mode)
    np.testing.assert_array_equal(y.view(np.uint32), case["y"].view(np.uint32))


# ---- GPU ------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(W8A8))
def test_gpu_w8a8_matches_fixture(hip, name):
    case = W8A8[name]
    m, k, n = dims(case, "m", "k", "n")
    packed = hip.w8a8_prepack(hip.DeviceBuffer.from_array(case["blob"]), k, n)
    xd = hip.DeviceBuffer.from_array(case["x"])
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, xd, packed, m, k, n, ws)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    raw = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_gemm(raw, q, s, packed, m, k, n, hip.EPI_RAW)
    hip.sync()
    np.testing.assert_array_equal(s.read(np.float32, m).view(np.uint32), case["s"].view(np.uint32))
    np.testing.assert_array_equal(raw.read(np.int32, m * n).reshape(m, n), case["acc"])
    got = y.read(np.float32, m * n).reshape(m, n)
    np.testing.assert_array_equal(got.view(np.uint32), case["y"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(F16))
def test_gpu_f16_matches_fixture(hip, name):
    case = F16[name]
    m, k, n, channels, mode = dims(case, "m", "k", "n", "channels", "mode")
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(case["w"]), k, n)
    bias = case.get("bias")
    bd = hip.DeviceBuffer.from_array(bias) if bias is not None else None
    out_elems = case["y"].size
    y = hip.DeviceBuffer(out_elems * 4)
    hip.f16_gemm(y, hip.DeviceBuffer.from_array(case["x"]), packed, bd, m, k, n, channels, mode)
    hip.sync()
    got = y.read(np.float32, out_elems).reshape(case["y"].shape)
    _, v, wk = f16_reference(case)
    absdot = np.abs(case["x"].astype(np.float16).astype(np.float64)) @ np.abs(wk)
    if mode == 3:
        absdot = absdot.T[:channels]
    bias_abs = 0.0 if bias is None else (np.abs(bias)[:, None] if mode == 3 else np.abs(bias)[None, :])
    assert_f16_close(got, case["y"], v, bias_abs, absdot, k)
