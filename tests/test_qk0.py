"""Opcodes 2/3/4: GEMM on Q4_0 / Q8_0 / IQ4_NL super-block weights.

The reference dequantizes each 256-weight super-block with HVX instructions
(reference src/dsp/ops/mat_mul.c:330-530) into the permuted fp16 layout of
opcode 1 and runs the F16 core.  The oracle restates the element order that
those instructions produce (oracle/htp_oracle.c, oracle_qk0_value).  It is
pinned here by a numpy model of the instructions:

- vshuff(hi, lo, -2) interleaves the halfwords of its two sources (what the
  shuffle instruction is for);
- vlut16 sends even source bytes to its low result and odd bytes to its high
  result, vunpack keeps byte order, vror / vlalign rotate and align bytes;
- run through the reference's single-group paths (mat_mul.c:282-329) this
  model reproduces ggml's published Q4_0 / IQ4_NL / Q8_0 group order, while a
  vlut16 that keeps byte order does not;
- run through the super-block paths (:394-427, :494-527) the same model
  equals oracle_qk0_value for every position.

Parity remains unpinned against the sd.cpp packer (absent from the reference)
and the qf16 rounding of value*scale (modelled as one binary16 rounding).
"""
import numpy as np
import pytest

import htp_ops as h
from tolerances import assert_f16_close, f16_abs_dot

TYPES = [(h.GGML_Q4_0, "q4_0"), (h.GGML_Q8_0, "q8_0"), (h.GGML_IQ4_NL, "iq4_nl")]
OPCODE = {h.GGML_Q4_0: 2, h.GGML_Q8_0: 3, h.GGML_IQ4_NL: 4}
BLOCK_BYTES = {h.GGML_Q4_0: 144, h.GGML_Q8_0: 272, h.GGML_IQ4_NL: 144}
# ggml's published IQ4_NL code book (kvalues_iq4nl)
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int32)


# ---- HVX instruction model (128-byte vectors) -----------------------------------

def lut_table(values):
    """A vlut16 table register: entry e at halfword 2e (the reference's
    q4_0_to_fp16_lut / iq4_nl_to_fp16_lut layout, mat_mul.c:30-37)."""
    t = np.zeros(64, np.float16)
    t[0:32:2] = np.asarray(values, np.float16)
    return t


def vlut16(src, table, keep_order=False):
    """Q6_Wh_vlut16_VbVhR_nomatch with R = 0: (lo, hi), 64 halfwords each."""
    idx = src.astype(np.int64) & 15
    if keep_order:  # the alternative model the group-order check must reject
        return table[idx[:64] * 2], table[idx[64:] * 2]
    return table[idx[0::2] * 2], table[idx[1::2] * 2]


def vshuff_h(hi, lo):
    """Q6_W_vshuff_VVR(hi, lo, -2): halfwords interleaved, lo first."""
    out = np.empty(128, hi.dtype)
    out[0::2], out[1::2] = lo, hi
    return out[:64], out[64:]


def vror(v, r):
    return np.roll(v, -r)


def vlalign(u, v, r):
    return np.concatenate([v[128 - r:], u[:128 - r]])


def vunpack_b(v):
    w = v.view(np.int8).astype(np.int16)
    return w[:64], w[64:]


def vmpy_hf(a, b):
    """qf16 multiply then conversion to IEEE half, modelled as one rounding."""
    return (a.astype(np.float32) * b.astype(np.float32)).astype(np.float16)


def single_group(window, scale_bits, kind, keep_order=False):
    """Model of dequantize_single_q4_0_group / _q8_0_group (mat_mul.c:282-329);
    `window` holds the 128 bytes from the group's quants on."""
    vs = np.zeros(64, np.float16)
    vs[0] = np.uint16(scale_bits).view(np.float16)
    v_scales = vlut16(np.zeros(128, np.uint8), vs)[0]
    if kind == "q8_0":
        return vmpy_hf(vunpack_b(window)[0].astype(np.float16), v_scales)[:32]
    lo, hi = window, window >> 4
    v_quants = vlalign(hi, vror(lo, 16), 16)
    table = lut_table(np.arange(16) - 8 if kind == "q4_0" else IQ4NL)
    vlo, vhi = vlut16(v_quants, table, keep_order)
    return vmpy_hf(vshuff_h(vhi, vlo)[0], v_scales)[:32]


def super_block(block, kind):
    """Model of the super-block loops (mat_mul.c:394-427 and :494-527): 256 halves."""
    scales = block[:16].view(np.float16)
    table_s = np.zeros(64, np.float16)
    table_s[0:16:2] = scales  # vunpack of the 8 halfword scales into words
    idx0 = np.array(([0, 2] * 32) + ([1, 3] * 32), np.uint8)
    s0, s1 = vlut16(idx0, table_s)
    s2, s3 = vlut16(idx0 + 4, table_s)
    if kind == "q8_0":
        q = block[16:272]
        v0, v1 = vunpack_b(q[:128])
        v2, v3 = vunpack_b(q[128:])
        vals = [v.astype(np.float16) for v in (v0, v1, v2, v3)]
    else:
        qs = block[16:144]
        table = lut_table(np.arange(16) - 8 if kind == "q4_0" else IQ4NL)
        q0 = vlut16(qs, table)
        q1 = vlut16(qs >> 4, table)
        vals = [q0[0], q0[1], q1[0], q1[1]]
    return np.concatenate([vmpy_hf(v, s) for v, s in zip(vals, (s0, s1, s2, s3))])


# ---- ggml's published group formats -------------------------------------------------

def ggml_group(qs, d, kind):
    d = np.float32(np.uint16(d).view(np.float16))
    if kind == "q8_0":
        q = qs[:32].view(np.int8).astype(np.int32)
    else:
        nib = np.concatenate([qs[:16] & 15, qs[:16] >> 4]).astype(np.int32)
        q = nib - 8 if kind == "q4_0" else IQ4NL[nib]
    return (q.astype(np.float32) * d).astype(np.float16)


def random_scale_bits(rng, count):
    # positive and negative normal fp16 scales across several binades
    mant = rng.integers(0, 1024, count)
    exp = rng.integers(5, 20, count)
    sign = rng.integers(0, 2, count)
    return ((sign << 15) | (exp << 10) | mant).astype(np.uint16)


@pytest.mark.parametrize("kind", ["q4_0", "iq4_nl", "q8_0"])
def test_model_single_group_is_ggml_order(kind):
    rng = np.random.default_rng(5)
    for _ in range(20):
        window = rng.integers(0, 256, 128).astype(np.uint8)
        d = random_scale_bits(rng, 1)[0]
        got = single_group(window, d, kind)
        np.testing.assert_array_equal(got.view(np.uint16), ggml_group(window, d, kind).view(np.uint16))


@pytest.mark.parametrize("kind", ["q4_0", "iq4_nl"])
def test_model_rejects_order_keeping_vlut16(kind):
    rng = np.random.default_rng(6)
    window = rng.integers(0, 256, 128).astype(np.uint8)
    d = np.float16(1.0).view(np.uint16)
    got = single_group(window, d, kind, keep_order=True)
    assert not np.array_equal(got, ggml_group(window, d, kind))


@pytest.mark.parametrize("wtype,kind", TYPES)
def test_oracle_matches_super_block_model(orc, wtype, kind):
    rng = np.random.default_rng(wtype)
    bb = BLOCK_BYTES[wtype]
    assert orc.qk0_block_bytes(wtype) == bb
    for _ in range(8):
        block = rng.integers(0, 256, bb).astype(np.uint8)
        block[:16] = random_scale_bits(rng, 8).view(np.uint8)
        model = super_block(block, kind).view(np.uint16)
        got = np.array([orc.qk0_value(block, j, wtype) for j in range(256)], np.uint16)
        np.testing.assert_array_equal(got, model)


@pytest.mark.parametrize("wtype,kind", TYPES)
def test_oracle_scale_one_gives_codes(orc, wtype, kind):
    """Scale 1.0 everywhere: every value is its code exactly, each code once
    per nibble/byte slot."""
    bb = BLOCK_BYTES[wtype]
    block = np.zeros(bb, np.uint8)
    block[:16] = np.full(8, 1.0, np.float16).view(np.uint8)
    if wtype == h.GGML_Q8_0:
        block[16:] = np.arange(256, dtype=np.int64).astype(np.uint8)
        expect = np.arange(256).astype(np.uint8).view(np.int8).astype(np.float16)
    else:
        block[16:] = np.arange(128, dtype=np.uint8)  # byte b: low nibble b%16, high nibble b//16 % 16
        codes = np.arange(16) - 8 if wtype == h.GGML_Q4_0 else IQ4NL
        b = np.arange(128)
        expect = np.concatenate([codes[b[0::2] % 16], codes[b[1::2] % 16], codes[(b[0::2] // 16) % 16],
                                 codes[(b[1::2] // 16) % 16]]).astype(np.float16)
    got = orc.qk0_dequant(np.tile(block, 4), 32, 32, wtype).view(np.float16)  # 4 super-blocks: one 32x32 tile
    for b in range(4):
        np.testing.assert_array_equal(got[b * 256:(b + 1) * 256], expect)


def test_oracle_dequant_layout_and_rejects(orc):
    """k*n/256 super-blocks, block b at positions [256b, 256b+256)."""
    k, n = 64, 96
    rng = np.random.default_rng(9)
    blocks = rng.integers(0, 256, k * n // 256 * 272).astype(np.uint8)
    blocks.reshape(-1, 272)[:, :16] = random_scale_bits(rng, k * n // 256 * 8).view(np.uint8).reshape(-1, 16)
    img = orc.qk0_dequant(blocks, k, n, h.GGML_Q8_0)
    for b in (0, 5, k * n // 256 - 1):
        blk = blocks[b * 272:(b + 1) * 272]
        np.testing.assert_array_equal(img[b * 256:(b + 1) * 256],
                                      [orc.qk0_value(blk, j, h.GGML_Q8_0) for j in range(256)])
    for bad in ((48, 64, h.GGML_Q8_0), (64, 48, h.GGML_Q8_0), (64, 64, 3)):
        with pytest.raises(ValueError):
            orc.qk0_dequant(np.zeros(64 * 64 * 2, np.uint8), *bad)


# ---- executor validation (host only) ---------------------------------------------------

@pytest.fixture(scope="module")
def bufs():
    big = h.RpcBuffer(1 << 20)
    unmapped = h.RpcBuffer(4096, map_it=False)
    yield big, unmapped
    for b in (big, unmapped):
        b.free()


@pytest.mark.parametrize("op", [2, 3, 4])
def test_qk0_executor_codes(bufs, op):
    """Reference op_executor.cc:771-800 and mat_mul.c:1604-1613: every failure is -1."""
    big, unmapped = bufs
    ok = [(big.fd, 0), (big.fd, 4096), (big.fd, 65536)]
    assert h.execute(op, h.matmul_params(*ok, 4, 64, 64)[:91])[0] == -1
    for i in range(3):
        a = list(ok)
        a[i] = (unmapped.fd, 0)
        assert h.execute(op, h.matmul_params(*a, 4, 64, 64))[0] == -1
        a = list(ok)
        a[i] = (big.fd, a[i][1] + 64)
        assert h.execute(op, h.matmul_params(*a, 4, 64, 64))[0] == -1
    for m, k, n in ((0, 64, 64), (4, 0, 64), (4, 64, 0), (-4, 64, 64), (4, 48, 64), (4, 64, 48), (4, -64, 64)):
        assert h.execute(op, h.matmul_params(*ok, m, k, n))[0] == -1
    # weight region past the end of the buffer
    assert h.execute(op, h.matmul_params(ok[0], ok[1], (big.fd, (1 << 20) - 4096), 4, 256, 256))[0] == -1


def test_qk0_sizes():
    assert h.qk0_weight_bytes(4096, 14336, h.GGML_Q4_0) == 4096 * 14336 // 256 * 144
    assert h.qk0_weight_bytes(4096, 14336, h.GGML_Q8_0) == 4096 * 14336 // 256 * 272
    assert h.qk0_weight_bytes(48, 64, h.GGML_Q4_0) == 0
    assert h.qk0_weight_bytes(64, 64, 3) == 0


# ---- GPU parity ---------------------------------------------------------------------------

def random_blocks(rng, k, n, wtype, scale_lo=-12, scale_hi=-6):
    """Super-blocks with random codes and fp16 scales 2^[scale_lo, scale_hi)."""
    bb = BLOCK_BYTES[wtype]
    nb = k * n // 256
    blocks = rng.integers(0, 256, nb * bb).astype(np.uint8).reshape(nb, bb)
    sc = (rng.uniform(1.0, 2.0, nb * 8) * 2.0 ** rng.integers(scale_lo, scale_hi, nb * 8))
    sc *= np.where(rng.integers(0, 2, nb * 8) == 1, -1.0, 1.0)
    blocks[:, :16] = sc.astype(np.float16).view(np.uint8).reshape(nb, 16)
    return blocks.ravel()


def unpermute(perm_bits, k, n):
    """Permuted fp16 image -> W [k][n] (float64) for the tolerance bound."""
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    idx = ((nn // 32) * (k // 32) + kk // 32) * 1024 + ((kk % 32) // 2) * 64 + (nn % 32) * 2 + kk % 2
    return perm_bits[idx].view(np.float16).astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,kind", TYPES)
@pytest.mark.parametrize("k,n", [(32, 32), (256, 96), (1536, 320)])
def test_qk0_prepack_bit_exact(hip, orc, wtype, kind, k, n):
    rng = np.random.default_rng(k + n + wtype)
    blocks = random_blocks(rng, k, n, wtype)
    img = orc.qk0_dequant(blocks, k, n, wtype)
    got = hip.qk0_prepack(hip.DeviceBuffer.from_array(blocks), k, n, wtype)
    ref = hip.f16_prepack(hip.DeviceBuffer.from_array(img), k, n)
    hip.sync()
    np.testing.assert_array_equal(got.read(np.uint16, k * n), ref.read(np.uint16, k * n))


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,kind", TYPES)
@pytest.mark.parametrize("m,k,n,scale_lo,scale_hi", [
    (1, 4096, 1024, -12, -6),    # one row: the whole-K ring kernel
    (1, 1536, 320, -12, -6),     # one row, K shorter than the waves cover
    (1, 4128, 64, -12, -6),      # one row, K past the ring kernels: split-K
    (2, 4096, 1024, -12, -6),    # two rows: the few-row ring kernel
    (16, 4096, 512, -12, -6),    # sixteen rows
    (5, 1536, 320, -12, -6),     # n % 64 != 0: the split-K path
    (5, 1536, 384, -12, -6),     # 64-column workgroups, K shorter than the waves cover
    (16, 96, 64, -12, -6),       # full 16 rows, k-blocks fewer than the waves
    (7, 32, 128, -12, -6),       # a single k-block
    (3, 4160, 64, -12, -6),      # few rows, K past the ring kernels: split-K
    (3, 512, 128, -24, -20),     # scales near the fp16 subnormal range: subnormal weights
    (1, 512, 128, -24, -20),
])
def test_qk0_direct_matches_prepacked(hip, orc, wtype, kind, m, k, n, scale_lo, scale_hi):
    """Few rows straight from the blocks: within the F16 bound of the oracle,
    and, where both take the split-K path (k > 4096), equal to the F16 path
    on the prepacked image bit for bit (same fp16 weights, same summation
    order)."""
    rng = np.random.default_rng(m * 7 + k + n + wtype)
    blocks = random_blocks(rng, k, n, wtype, scale_lo, scale_hi)
    x = orc.normal(m * k, 0, 1, m + n).reshape(m, k)
    bd, xd = hip.DeviceBuffer.from_array(blocks), hip.DeviceBuffer.from_array(x)
    ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, n), 256))
    y1, y2 = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4)
    hip.qk0_gemm(y1, xd, bd, m, k, n, wtype, ws)
    packed = hip.qk0_prepack(bd, k, n, wtype)
    hip.f16_gemm(y2, xd, packed, None, m, k, n, n, 0, workspace=ws)
    hip.sync()
    if k > 4096:
        np.testing.assert_array_equal(y1.read(np.uint32, m * n), y2.read(np.uint32, m * n))
    ref = orc.f16_gemm_epilogue(x, orc.qk0_dequant(blocks, k, n, wtype), None, m, k, n, n, 0)
    img = orc.qk0_dequant(blocks, k, n, wtype)
    assert_f16_close(y1.read(np.float32, m * n).reshape(m, n), ref, ref, 0.0, f16_abs_dot(x, unpermute(img, k, n)), k)


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,kind", TYPES)
@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("m,k,n", [(1, 4096, 1024), (16, 512, 256), (77, 768, 3072), (300, 256, 576)])
def test_qk0_opcode_end_to_end(hip, orc, wtype, kind, device, m, k, n):
    rng = np.random.default_rng(m + k + n + wtype)
    x = orc.normal(m * k, 0, 1, m + k).reshape(m, k)
    blocks = random_blocks(rng, k, n, wtype)
    img = orc.qk0_dequant(blocks, k, n, wtype)
    ref = orc.f16_gemm_epilogue(x, img, None, m, k, n, n, 0)
    out = h.RpcBuffer(m * n * 4, device=device)
    act = h.RpcBuffer(m * k * 4, device=device)
    wgt = h.RpcBuffer(blocks.nbytes, device=device)
    try:
        act.write(x)
        wgt.write(blocks)
        rc, _ = h.execute(OPCODE[wtype], h.matmul_params((out.fd, 0), (act.fd, 0), (wgt.fd, 0), m, k, n))
        assert rc == 0, h.last_error()
        got = out.read(np.float32, m * n).reshape(m, n)
        assert_f16_close(got, ref, ref, 0.0, f16_abs_dot(x, unpermute(img, k, n)), k)
        # a rewrite of the weight buffer is seen by the next call (cache keyed on the contents)
        blocks2 = random_blocks(rng, k, n, wtype)
        wgt.write(blocks2)
        ref2 = orc.f16_gemm_epilogue(x, orc.qk0_dequant(blocks2, k, n, wtype), None, m, k, n, n, 0)
        rc, _ = h.execute(OPCODE[wtype], h.matmul_params((out.fd, 0), (act.fd, 0), (wgt.fd, 0), m, k, n))
        assert rc == 0, h.last_error()
        got2 = out.read(np.float32, m * n).reshape(m, n)
        assert_f16_close(got2, ref2, ref2, 0.0,
                         f16_abs_dot(x, unpermute(orc.qk0_dequant(blocks2, k, n, wtype), k, n)), k)
    finally:
        for b in (out, act, wgt):
            b.free()
