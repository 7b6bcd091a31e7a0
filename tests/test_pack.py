"""Host packers of the product library against the oracle and the reference formats (CPU)."""
import numpy as np
import pytest

import htp_ops as h


@pytest.mark.parametrize("k,n", [(32, 64), (96, 128), (768, 3072)])
def test_pack_constants_matches_oracle(orc, k, n):
    w = orc.int8_uniform(n * k, -128, 127, k + n).reshape(n, k)
    sw = orc.uniform(n, 1e-4, 1e-3, 3)
    inv = orc.uniform(k, 0.5, 2.0, 4)
    sums = np.random.default_rng(5).integers(-2**30, 2**30, n).astype(np.int32)
    for kwargs in ({}, {"sums": sums}, {"inv": inv}, {"sums": sums, "inv": inv, "signature": 0x1234abcd}):
        ours = h.pack_constants(w, sw, **kwargs)
        ref = orc.pack_blob(w, sw, **kwargs)
        assert np.array_equal(ours, ref)
        assert orc.check_header(ours, k, n) == 0


def test_pack_constants_rejects_bad_shapes():
    with pytest.raises(h.HtpOpsError):
        h.pack_constants(np.zeros((32, 64), np.int8), np.ones(32, np.float32))   # n % 64
    with pytest.raises(h.HtpOpsError):
        h.pack_constants(np.zeros((64, 48), np.int8), np.ones(64, np.float32))   # k % 32


def test_permute_f16_matches_oracle(orc):
    k, n = 96, 128
    w = np.random.default_rng(0).integers(0, 65536, (k, n)).astype(np.uint16)
    assert np.array_equal(h.permute_f16(w), orc.f16_permute(w))


def test_quantize_weights_closed_form():
    rng = np.random.default_rng(1)
    n, k = 64, 96
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    w[3] = 0.0
    q, sw = h.quantize_weights(w)
    amax = np.abs(w).max(axis=1)
    expect_sw = np.where(amax > 0, (amax / np.float32(127)).astype(np.float32), np.float32(1))
    assert np.array_equal(sw, expect_sw)
    assert np.array_equal(q, np.clip(np.rint(w / sw[:, None]), -127, 127).astype(np.int8))
    assert (np.abs(q).max(axis=1)[np.arange(n) != 3] == 127).all()
    # dequantization error within half a step
    assert np.all(np.abs(q * sw[:, None] - w) <= sw[:, None] * 0.5 + 1e-12)


def test_fnv1a64_known_values():
    assert h.lib().htp_ops_fnv1a64(None, 0) == 0xcbf29ce484222325
    data = np.frombuffer(b"a", np.uint8)
    assert h.lib().htp_ops_fnv1a64(data.ctypes.data, 1) == 0xaf63dc4c8601ec8c


def test_pack_f16_equals_quantize_then_pack(orc):
    """FP16 source weights: exact widening (normals, subnormals, signed zero),
    per-channel quantization with and without a smoothing vector, sums of the
    quantized weights and the FNV-1a signature of the fp16 bytes, byte for
    byte against the separate steps (the oracle packer for the blob)."""
    rng = np.random.default_rng(7)
    n, k = 128, 96
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    w[5, :7] = np.array([0.0, -0.0, 6e-8, -6e-8, 2.0 ** -20, 65504.0, -65504.0], np.float16)  # subnormals, extremes
    w[9] = 0.0
    inv = orc.uniform(k, 0.5, 2.0, 8)
    for smoothing in (None, inv):
        blob = h.pack_f16(w, inv=smoothing)
        q, sw = h.quantize_weights(w.astype(np.float32), inv=smoothing)
        sig = h.lib().htp_ops_fnv1a64(w.ctypes.data, w.nbytes)
        ref = orc.pack_blob(q, sw, inv=smoothing, signature=sig)
        assert np.array_equal(blob, ref)
        assert int(np.frombuffer(blob[40:48].tobytes(), np.uint64)[0]) == sig
    # the widening is exact: numpy's float16 -> float32 conversion is the reference
    bits = np.arange(65536, dtype=np.uint16)
    finite = np.isfinite(bits.view(np.float16))
    wide = bits[finite][: (finite.sum() // (64 * 32)) * 64 * 32].reshape(64, -1)
    kk = wide.shape[1] // 32 * 32
    wide = np.ascontiguousarray(wide[:, :kk])
    blob = h.pack_f16(wide.view(np.float16))
    q, sw = h.quantize_weights(wide.view(np.float16).astype(np.float32))
    assert np.array_equal(blob, orc.pack_blob(q, sw, signature=h.lib().htp_ops_fnv1a64(wide.ctypes.data, wide.nbytes)))


def test_pack_f16_rejects_bad_shapes():
    with pytest.raises(h.HtpOpsError):
        h.pack_f16(np.zeros((32, 64), np.float16))   # n % 64
    with pytest.raises(h.HtpOpsError):
        h.pack_f16(np.zeros((64, 48), np.float16))   # k % 32
