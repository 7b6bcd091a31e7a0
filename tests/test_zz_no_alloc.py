"""hb_w8a8_linear_noalloc (the entry point with a static device workspace)
against hb_w8a8_linear on the same inputs: bit-exact, on calls in a row with
the second input smaller, through the C ABI."""
import numpy as np
import pytest

import htp_ops as h

pytestmark = pytest.mark.gpu


def _case(orc, m, k, n, seed):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    x[:, np.random.default_rng(seed).choice(k, max(1, k // 100), replace=False)] *= 20.0
    w = orc.int8_uniform(n * k, -127, 127, seed + 1).reshape(n, k)
    sw = orc.uniform(n, 1e-4, 1e-3, seed + 2)
    inv = orc.uniform(k, 0.5, 2.0, seed + 3)
    blob = orc.pack_blob(w, sw, inv=inv, signature=seed)
    packed = h.w8a8_prepack(h.DeviceBuffer.from_array(blob), k, n)
    return x, blob, packed


def _noalloc(y, x, packed, m, k, n, epilogue=h.EPI_SCALE):
    return h.lib().hb_w8a8_linear_noalloc(y.ptr, x.ptr, packed.ptr, m, k, n, epilogue, None)


@pytest.mark.parametrize("shapes", [
    [(2048, 1536, 3072), (300, 768, 1024)],   # quantize + tiled GEMM, then a smaller tiled case
    [(77, 768, 3072), (1, 4096, 2048)],       # one-launch small kernel, then the fused one-row kernel
    [(4096, 6144, 1536), (16, 4096, 4096)],   # the largest C3 layer (25 MB workspace), then few rows
])
def test_noalloc_matches_linear(hip, orc, shapes):
    lib = h.lib()
    for epi in (h.EPI_SCALE, h.EPI_SCALE_GELU):
        for i, (m, k, n) in enumerate(shapes):
            x, blob, packed = _case(orc, m, k, n, seed=m + k + n + i)
            xd = h.DeviceBuffer.from_array(x)
            ws = h.DeviceBuffer(h.w8a8_workspace_bytes(m, k))
            y_ref, y_na = h.DeviceBuffer(m * n * 4), h.DeviceBuffer(m * n * 4)
            y_na.fill(0x5A)
            h.w8a8_linear(y_ref, xd, packed, m, k, n, ws, epilogue=epi)
            assert _noalloc(y_na, xd, packed, m, k, n, epi) == 0, h.last_error()
            h.sync()
            np.testing.assert_array_equal(y_na.read(np.uint32, m * n), y_ref.read(np.uint32, m * n))
            if epi == h.EPI_SCALE:  # and the oracle, bit for bit
                ref = orc.linear(x, blob, k, n)
                np.testing.assert_array_equal(y_na.read(np.uint32, m * n).reshape(m, n), ref.view(np.uint32))
            for b in (xd, ws, y_ref, y_na, packed):
                b.free()


def test_noalloc_rejects_oversized(hip, orc):
    m, k, n = 4096, 8192, 64
    assert h.w8a8_workspace_bytes(m, k) > 32 << 20
    x, _, packed = _case(orc, 16, k, n, seed=9)
    xd = h.DeviceBuffer(m * k * 4)
    y = h.DeviceBuffer(m * n * 4)
    rc = _noalloc(y, xd, packed, m, k, n)
    assert rc == h.HB_E_INVAL
    assert b"static workspace" in h.lib().hb_last_error()
