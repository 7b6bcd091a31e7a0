"""Opcodes 15 / 16 / 1 through the drop-in boundary on the GPU, against the oracle.

Requests go through execute_op_simple, the mailbox channel thread and the
direct W16 entry points, with host (rpcmem) and HBM-resident tensors.
W8A8 outputs are compared bit-exactly; F16 within 2e-3 of the fp16-rounded
magnitude (see tests/test_gpu_kernels.py for the bound's derivation).
"""
import ctypes
import struct
import time

import numpy as np
import pytest

import htp_ops as h
from tolerances import assert_f16_close, f16_abs_dot

pytestmark = pytest.mark.gpu


def f16_weight(orc, k, n, seed):
    w = orc.normal(k * n, 0, 0.02, seed).reshape(k, n).astype(np.float16)
    return w, h.permute_f16(w.view(np.uint16))


def w8a8_inputs(orc, m, k, n, seed, inv=False, sums=False):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    w = orc.int8_uniform(n * k, -127, 127, seed + 1).reshape(n, k)
    sw = orc.uniform(n, 1e-4, 1e-3, seed + 2)
    invv = orc.uniform(k, 0.5, 2.0, seed + 3) if inv else None
    sumv = np.random.default_rng(seed).integers(-2**20, 2**20, n).astype(np.int32) if sums else None
    return x, h.pack_constants(w, sw, sums=sumv, inv=invv, signature=seed)


def rpc(nbytes, device):
    return h.RpcBuffer(nbytes, device=device)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("m,k,n", [
    (77, 768, 3072),   # C1: the one-launch small kernel (quantizes its own rows)
    (1, 4096, 1024),   # one row: quantization inside the weight stream
    (3, 4096, 2048),   # 2-4 rows fused
    (16, 4096, 4096),  # few rows: quantize + decode GEMM
    (64, 1536, 1024),  # 5-128 rows, short K
    (300, 96, 512),    # quantize + tiled GEMM
    (77, 8192, 1024),  # 33-256 rows, long K: split-K over int32 slices in the executor's workspace
])
def test_opcode15_bit_exact(hip, orc, device, m, k, n):
    x, blob = w8a8_inputs(orc, m, k, n, seed=m + n, inv=True, sums=True)
    out, act, cst = rpc(m * n * 4 + 256, device), rpc(m * k * 4 + 512, device), rpc(blob.nbytes + 1024, device)
    act.write(x, 512)
    cst.write(blob, 1024)
    rc, payload = h.execute(15, h.w8a8_params((out.fd, 256), (act.fd, 512), (cst.fd, 1024), m, k, n))
    assert rc == 0, h.last_error()
    y = out.read(np.float32, m * n, 256).reshape(m, n)
    ref = orc.linear(x, blob, k, n)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    elapsed = struct.unpack_from("<i", payload, 36)[0]
    assert elapsed >= 0


def test_opcode15_profile_modes(hip, orc):
    m, k, n = 64, 256, 512
    x, blob = w8a8_inputs(orc, m, k, n, seed=3)
    out, act, cst = rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(blob.nbytes, False)
    act.write(x)
    cst.write(blob)
    ref = orc.linear(x, blob, k, n)
    for mode in (1, 2, 3):
        payload = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n) + h.w8a8_profile(mode)
        rc, after = h.execute(15, payload)
        assert rc == 0
        prof = h.unpack_w8a8_profile(after[40:])
        assert prof["mode"] == mode
        assert prof["hmx_ticks"] > 0 and prof["activation_ticks"] > 0
        if mode == 2:
            # MAC (the accumulating GEMM) and readout (the separate epilogue launch) timed apart
            assert prof["mac_ticks"] > 0 and prof["readout_ticks"] > 0
            assert prof["mac_ticks"] + prof["readout_ticks"] == prof["hmx_ticks"]
            assert prof["output_ticks"] == 0
        if mode == 3:
            assert prof["reserved"] == gemm_tile(m, k, n)
        assert np.array_equal(out.read(np.float32, m * n).reshape(m, n), ref)


def gemm_tile(m, k, n):
    """rows | columns << 16 of the tile hb_w8a8_gemm runs for this shape."""
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    assert h.lib().hb_w8a8_gemm_tile(m, k, n, ctypes.byref(bm), ctypes.byref(bn)) >= -2
    return bm.value | (bn.value << 16)


def test_opcode15_profile_mode3_reports_the_tile_that_ran(hip, orc):
    """Mode 3's reserved field holds the GEMM's tile rows | columns << 16:
    256 x 192 streaming tiles at the headline shape, 16-row tiles for few rows."""
    assert gemm_tile(4096, 1536, 6144) == 256 | (192 << 16)
    assert gemm_tile(4, 4096, 14336) == 16 | (16 << 16)
    for m, k, n in ((4096, 1536, 6144), (4, 4096, 4096)):
        x, blob = w8a8_inputs(orc, m, k, n, seed=5)
        out, act, cst = rpc(m * n * 4, True), rpc(m * k * 4, True), rpc(blob.nbytes, True)
        act.write(x)
        cst.write(blob)
        payload = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n) + h.w8a8_profile(3)
        rc, after = h.execute(15, payload)
        assert rc == 0
        prof = h.unpack_w8a8_profile(after[40:])
        assert prof["mode"] == 3 and prof["reserved"] == gemm_tile(m, k, n)
        for b in (out, act, cst):
            b.free()


def test_opcode15_cpu_control_variant(hip, orc):
    """Raw accumulator planes over the output + row scales + one batch."""
    m, k, n = 77, 128, 128
    x, blob = w8a8_inputs(orc, m, k, n, seed=9)
    out, act, cst, ctl = (rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(blob.nbytes, False),
                          rpc(17536, False))
    act.write(x)
    cst.write(blob)
    ctl.write(np.zeros(17536, np.uint8))
    payload = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n) + struct.pack("<ii", ctl.fd, 0)
    rc, _ = h.execute(15, payload)
    assert rc == 0
    inv = np.ones(k, np.float32)
    u, s = orc.quantize(x, inv)
    acc = orc.accumulate(u, blob, k, n)
    assert np.array_equal(out.read(np.uint8, m * n * 4), orc.planes(acc))
    c = ctl.read(np.uint8, 17536)
    assert struct.unpack_from("<I", c, 0)[0] == 1                      # produced
    assert np.array_equal(np.frombuffer(c[128:128 + 4 * m].tobytes(), np.float32), s)
    assert struct.unpack_from("<4i", c, 16512) == (0, m, 0, n // 64)


@pytest.mark.parametrize("m,k,n,flags,resident,rows,wcols,out_dev,ctl_dev", [
    # activation-first plan: min(2 MB, VTCM beside one slab) / (64 k) = 5 slabs of 64 rows at k = 6144;
    # 13 resident weight slabs beside them (reference linear_w8a8.c:380-388)
    (700, 6144, 256, 0, 0, 320, 13, False, False),
    # weight-first (all 512 columns resident): the caller's 200 rows -> 3 slabs (linear_w8a8.c:373-379)
    (700, 256, 512, 1, 200, 192, 8, True, False),
    # HBM-resident output and control block
    (700, 6144, 256, 0, 0, 320, 13, True, True),
])
def test_opcode15_cpu_control_batches(hip, orc, m, k, n, flags, resident, rows, wcols, out_dev, ctl_dev):
    """The CPU-control variant publishes one batch per M chunk of the
    reference's plan; planes, scales and batch records of every chunk."""
    x, blob = w8a8_inputs(orc, m, k, n, seed=m + k)
    out, act, cst, ctl = (rpc(m * n * 4, out_dev), rpc(m * k * 4, False), rpc(blob.nbytes, False),
                          rpc(17536, ctl_dev))
    act.write(x)
    cst.write(blob)
    c0 = np.zeros(17536, np.uint8)
    struct.pack_into("<I", c0, 4, flags)
    struct.pack_into("<I", c0, 32, resident)
    struct.pack_into("<I", c0, 0, 99)  # stale progress from an earlier call
    ctl.write(c0)
    payload = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n) + struct.pack("<ii", ctl.fd, 0)
    rc, _ = h.execute(15, payload)
    assert rc == 0
    u, s = orc.quantize(x, np.ones(k, np.float32))
    assert np.array_equal(out.read(np.uint8, m * n * 4), orc.planes(orc.accumulate(u, blob, k, n)))
    c = ctl.read(np.uint8, 17536)
    nb = (m + rows - 1) // rows
    assert struct.unpack_from("<I", c, 0)[0] == nb                      # produced
    assert struct.unpack_from("<III", c, 8) == (8 << 20, rows, wcols)    # vtcm_bytes, activation_rows, weight_columns
    assert np.array_equal(np.frombuffer(c[128:128 + 4 * m].tobytes(), np.float32), s)
    for b in range(nb):
        assert struct.unpack_from("<4i", c, 16512 + 16 * b) == (b * rows, min(rows, m - b * rows), 0, n // 64)


def test_opcode15_weight_cache_follows_rewrites(hip, orc):
    m, k, n = 16, 256, 256
    x, blob1 = w8a8_inputs(orc, m, k, n, seed=21)
    _, blob2 = w8a8_inputs(orc, m, k, n, seed=22)
    out, act, cst = rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(blob1.nbytes, False)
    act.write(x)
    params = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n)
    for blob in (blob1, blob1, blob2, blob1):
        cst.write(blob)
        assert h.execute(15, params)[0] == 0
        ref = orc.linear(x, blob, k, n)
        assert np.array_equal(out.read(np.float32, m * n).reshape(m, n), ref)
    assert h.lib().htp_ops_amd_invalidate_weights(cst.fd) >= 1


@pytest.mark.parametrize("section", ["inverse", "scale", "weights"])
def test_opcode15_host_blob_rewritten_in_place(hip, orc, section):
    """The reference reads the constants on every call, so rewriting part of a
    host-resident blob in place (no map put, no invalidate call) must change
    the next result: the smoothing vector, the per-column scales, or one
    weight byte far from the blob's ends."""
    m, k, n = 8, 1536, 1024
    x, blob = w8a8_inputs(orc, m, k, n, seed=51, inv=True)
    out, act, cst = rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(blob.nbytes, False)
    act.write(x)
    cst.write(blob)
    params = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n)
    assert h.execute(15, params)[0] == 0
    assert np.array_equal(out.read(np.float32, m * n).reshape(m, n), orc.linear(x, blob, k, n))
    new = blob.copy()
    if section == "inverse":
        off = 128 + k * n + 8 * n
        new[off:off + 4 * k] = np.frombuffer(orc.uniform(k, 0.25, 4.0, 52).tobytes(), np.uint8)
    elif section == "scale":
        off = 128 + k * n
        new[off:off + 4 * n] = np.frombuffer(orc.uniform(n, 1e-3, 1e-2, 53).tobytes(), np.uint8)
    else:
        off = 128 + k * n // 2 + 4093
        new[off] = np.uint8((int(new[off]) + 77) & 0xff)
    # written straight into the rpcmem memory, as a caller does (the library sees no write)
    end = off + (4 * k if section == "inverse" else 4 * n if section == "scale" else 1)
    cst.host_view()[off:end] = new[off:end]
    assert h.execute(15, params)[0] == 0
    ref = orc.linear(x, new, k, n)
    assert not np.array_equal(ref, orc.linear(x, blob, k, n))
    assert np.array_equal(out.read(np.float32, m * n).reshape(m, n).view(np.uint32), ref.view(np.uint32))


def test_opcode15_large_host_blob_rewrites_in_every_share(hip, orc):
    """Blobs of 4 MiB and more are hashed in 1 MiB chunks spread over
    threads: one byte rewritten in place in the first, a middle and the last
    chunk is seen by the next call each time."""
    m, k, n = 8, 4096, 2048
    x, blob = w8a8_inputs(orc, m, k, n, seed=61)
    assert blob.nbytes >= 8 << 20
    out, act, cst = rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(blob.nbytes, False)
    act.write(x)
    cst.write(blob)
    params = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n)
    assert h.execute(15, params)[0] == 0
    cur = blob.copy()
    for off in (128 + 999, (5 << 20) + 12345, 128 + k * n - 7):
        cur[off] = np.uint8((int(cur[off]) + 101) & 0xff)
        cst.host_view()[off:off + 1] = cur[off:off + 1]
        assert h.execute(15, params)[0] == 0
        ref = orc.linear(x, cur, k, n)
        assert np.array_equal(out.read(np.float32, m * n).reshape(m, n).view(np.uint32), ref.view(np.uint32))


def test_opcode15_device_blob_header_after_cache_hit(hip, orc):
    """A cached device blob skips the header read-back; a rewrite with a bad
    header is still rejected (-3), and a good rewrite runs again."""
    m, k, n = 8, 128, 128
    x, blob = w8a8_inputs(orc, m, k, n, seed=31)
    out, act, cst = rpc(m * n * 4, True), rpc(m * k * 4, True), rpc(blob.nbytes, True)
    act.write(x)
    cst.write(blob)
    params = h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n)
    ref = orc.linear(x, blob, k, n)
    for _ in range(2):  # build, then a cache hit
        assert h.execute(15, params)[0] == 0
        assert np.array_equal(out.read(np.float32, m * n).reshape(m, n), ref)
    bad = blob.copy()
    bad[:4] ^= 0xFF  # magic
    cst.write(bad)
    assert h.execute(15, params)[0] == -3
    cst.write(blob)
    assert h.execute(15, params)[0] == 0
    assert np.array_equal(out.read(np.float32, m * n).reshape(m, n), ref)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("mode,channels", [(0, 768), (1, 768), (2, 768), (3, 700)])
def test_opcode16_modes(hip, orc, device, mode, channels):
    m, k, n = 77, 3072 if mode == 0 else 768, 768
    x = orc.normal(m * k, 0, 1, mode).reshape(m, k)
    w, perm = f16_weight(orc, k, n, 10 + mode)
    bias = orc.normal(channels, 0, 0.02, 20 + mode)
    out_elems = m * channels
    out, act, wgt, b = (rpc(out_elems * 4, device), rpc(m * k * 4, device), rpc(perm.nbytes, device),
                        rpc(channels * 4, device))
    act.write(x)
    wgt.write(perm)
    b.write(bias)
    rc, payload = h.execute(16, h.f16_epilogue_params((out.fd, 0), (act.fd, 0), (wgt.fd, 0), (b.fd, 0), m, k, n,
                                                      channels, mode))
    assert rc == 0, h.last_error()
    got = out.read(np.float32, out_elems)
    ref = orc.f16_gemm_epilogue(x, perm, bias, m, k, n, channels, mode)
    v = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
    absdot = f16_abs_dot(x, w)
    if mode == 3:
        got, v, bterm, absdot = got.reshape(channels, m), v.T[:channels], np.abs(bias)[:, None], absdot.T[:channels]
    else:
        got, bterm = got.reshape(m, n), np.abs(bias)[None, :]
    assert_f16_close(got, ref, v, bterm, absdot, k)
    assert struct.unpack_from("<i", payload, 52)[0] >= 0


def test_opcode1_and_direct_rpc(hip, orc):
    m, k, n = 32, 256, 512
    x = orc.normal(m * k, 0, 1, 31).reshape(m, k)
    w, perm = f16_weight(orc, k, n, 32)
    out, act, wgt = rpc(m * n * 4, False), rpc(m * k * 4, False), rpc(perm.nbytes, False)
    act.write(x)
    wgt.write(perm)
    ref = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
    absdot = f16_abs_dot(x, w)
    rc, payload = h.execute(1, h.matmul_params((out.fd, 0), (act.fd, 0), (wgt.fd, 0), m, k, n, with_elapsed=True))
    assert rc == 0
    assert_f16_close(out.read(np.float32, m * n).reshape(m, n), ref, ref, 0.0, absdot, k)
    assert struct.unpack_from("<i", payload, 92)[0] >= 0
    lib = h.lib()
    handle = ctypes.c_uint64()
    assert lib.htp_ops_open(b"", ctypes.byref(handle)) == 0
    assert lib.htp_ops_mat_mul_permuted_w16a32(handle, out.fd, 0, act.fd, 0, wgt.fd, 0, m, k, n) == h.AEE_EBADSTATE
    assert lib.htp_ops_init_backend(handle) == 0
    out.write(np.zeros(m * n, np.float32))
    assert lib.htp_ops_mat_mul_permuted_w16a32(handle, out.fd, 0, act.fd, 0, wgt.fd, 0, m, k, n) == 0
    y = out.read(np.float32, m * n)
    assert_f16_close(y.reshape(m, n), ref, ref, 0.0, absdot, k)
    ah, oh, orh = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    assert lib.htp_ops_mat_mul_permuted_w16a32_trace(handle, out.fd, 0, act.fd, 0, wgt.fd, 0, m, k, n,
                                                     ctypes.byref(ah), ctypes.byref(oh), ctypes.byref(orh)) == 0
    xb = np.ascontiguousarray(x)
    assert ah.value == lib.htp_ops_fnv1a64(xb.ctypes.data, xb.nbytes)
    assert oh.value == orh.value == lib.htp_ops_fnv1a64(y.ctypes.data, y.nbytes)
    assert lib.htp_ops_close(handle) == 0


def test_weight_cache_in_a_shared_buffer(hip, orc):
    """One HBM buffer holds a weight, activations and outputs.  Outputs written
    elsewhere in it keep the cached weight image (results unchanged); an
    output written over the weight's own bytes makes the next call use the
    new bytes."""
    m, k, n = 32, 64, 64
    rng = np.random.default_rng(41)
    x = rng.integers(-2, 3, (m, k)).astype(np.float32)
    w1 = rng.integers(-2, 3, (k, n)).astype(np.float16)
    w3 = rng.integers(-2, 3, (k, n)).astype(np.float16)
    p1, p3 = h.permute_f16(w1.view(np.uint16)), h.permute_f16(w3.view(np.uint16))
    ow, ow3, ox, oy = 0, 8192, 16384, 24576  # the weight's k*n*2 bytes = the m*n*4 output bytes
    buf = rpc(32768, True)
    buf.write(p1, ow)
    buf.write(p3, ow3)
    buf.write(x, ox)

    def matmul(out, wgt):
        rc, _ = h.execute(1, h.matmul_params((buf.fd, out), (buf.fd, ox), (buf.fd, wgt), m, k, n))
        assert rc == 0, h.last_error()

    matmul(oy, ow)
    y1 = buf.read(np.float32, m * n, oy)
    assert np.array_equal(y1.reshape(m, n), x @ w1.astype(np.float32))  # small integers: exact
    matmul(oy, ow)  # the output lands beside the weight: same result
    assert np.array_equal(buf.read(np.float32, m * n, oy), y1)
    matmul(ow, ow3)  # the output overwrites the first weight's bytes
    w2_perm = buf.read(np.uint16, k * n, ow)
    assert not np.array_equal(w2_perm, p1)
    matmul(oy, ow)  # must read the new bytes, not the cached image of the old ones
    ref = orc.f16_gemm_epilogue(x, w2_perm, None, m, k, n, n, 0)
    got = buf.read(np.float32, m * n, oy).reshape(m, n)
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(ref) + 1e-6)
    assert not np.allclose(got, y1.reshape(m, n))


def post(chan_view, requests, capacity, timeout=60.0):
    msg, offs = h.build_message(requests, capacity)
    chan_view[8:len(msg)] = np.frombuffer(bytes(msg[8:]), np.uint8)
    chan_view[:8] = 0
    chan_view[0] = 1
    t0 = time.time()
    while chan_view[1] != 1:
        assert time.time() - t0 < timeout
        time.sleep(0.0002)
    return bytearray(chan_view[:capacity].tobytes()), offs


def test_mailbox_chained_requests(hip, orc):
    """A W8A8 request whose output feeds an F16 request in the same message,
    then a map put and a repeat: requests run in order on one channel."""
    lib = h.lib()
    assert lib.open_dsp_session(3, 1) == 0
    lib.init_htp_backend()
    assert lib.htp_ops_session_is_initialized(lib.htp_ops_default_session()) == 1
    chan = h.RpcBuffer(4096)
    assert lib.create_htp_message_channel(chan.fd, 4096) == 0
    m, k, n, n2 = 77, 768, 768, 256
    x, blob = w8a8_inputs(orc, m, k, n, seed=41)
    w2, perm = f16_weight(orc, n, n2, 42)
    tensors = h.RpcBuffer(1 << 24)
    off_x, off_blob, off_y, off_w, off_z = 0, 1 << 20, 3 << 20, 4 << 20, 5 << 20
    tensors.write(x, off_x)
    tensors.write(blob, off_blob)
    tensors.write(perm, off_w)
    fd = tensors.fd
    r1 = h.compute_request(15, h.w8a8_params((fd, off_y), (fd, off_x), (fd, off_blob), m, k, n))
    r2 = h.compute_request(16, h.f16_epilogue_params((fd, off_z), (fd, off_y), (fd, off_w), (-1, 0), m, n, n2, n2, 1))
    put = struct.pack("<ii", 1, 0) + struct.pack("<i", fd)
    view = chan.host_view()
    for _ in range(2):
        done, offs = post(view, [(h.REQUEST_TYPE_OP_COMPUTE, r1), (h.REQUEST_TYPE_OP_COMPUTE, r2),
                                 (h.REQUEST_TYPE_RPCMEM_MAP, put)], 4096)
        assert [h.request_state(done, offs, i) for i in range(3)] == [0, 0, 0]
        y = tensors.read(np.float32, m * n, off_y).reshape(m, n)
        ref_y = orc.linear(x, blob, k, n)
        assert np.array_equal(y.view(np.uint32), ref_y.view(np.uint32))
        z = tensors.read(np.float32, m * n2, off_z).reshape(m, n2)
        ref_z = orc.f16_gemm_epilogue(ref_y, perm, None, m, n, n2, n2, 1)
        v = orc.f16_gemm_epilogue(ref_y, perm, None, m, n, n2, n2, 0)
        assert_f16_close(z, ref_z, v, 0.0, f16_abs_dot(ref_y, w2), n)
    assert lib.destroy_htp_message_channel() == 0
    lib.close_dsp_session()
    chan.free()
    tensors.free()


def test_test_ops_on_gpu_backend(hip):
    lib = h.lib()
    handle = ctypes.c_uint64()
    assert lib.htp_ops_open(b"", ctypes.byref(handle)) == 0
    assert lib.htp_ops_init_backend(handle) == 0
    scope = ctypes.c_int32()
    assert lib.htp_ops_test_ops(handle, ctypes.byref(scope)) == 0 and scope.value == 1
    assert lib.htp_ops_close(handle) == 0


def test_mailbox_device_requests_complete_once_per_message(hip, orc):
    """Several opcode-15 requests on HBM tensors in one message: the executor
    synchronises once for the message, yet every output is complete and
    every elapsed_us field is written when the completion flag is seen."""
    lib = h.lib()
    assert lib.open_dsp_session(3, 1) == 0
    lib.init_htp_backend()
    chan = h.RpcBuffer(4096)
    assert lib.create_htp_message_channel(chan.fd, 4096) == 0
    cases = [(1024, 1536, 3072, 61), (1, 4096, 2048, 62), (77, 768, 3072, 63), (300, 1536, 1536, 64)]
    bufs, reqs, refs = [], [], []
    for m, k, n, seed in cases:
        x, blob = w8a8_inputs(orc, m, k, n, seed=seed, inv=True)
        out, act, cst = rpc(m * n * 4, True), rpc(m * k * 4, True), rpc(blob.nbytes, True)
        act.write(x)
        cst.write(blob)
        bufs.append((out, act, cst))
        reqs.append((h.REQUEST_TYPE_OP_COMPUTE,
                     h.compute_request(15, h.w8a8_params((out.fd, 0), (act.fd, 0), (cst.fd, 0), m, k, n))))
        refs.append(orc.linear(x, blob, k, n))
    view = chan.host_view()
    for rep in range(2):
        for out, _, _ in bufs:
            out.write(np.zeros(out.nbytes // 4, np.float32))
        done, offs = post(view, reqs, 4096)
        assert [h.request_state(done, offs, i) for i in range(len(cases))] == [0] * len(cases)
        for i, ((m, k, n, _), (out, _, _), ref) in enumerate(zip(cases, bufs, refs)):
            got = out.read(np.float32, m * n).reshape(m, n)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, i)
            elapsed = struct.unpack_from("<i", h.request_data(done, offs, i), 4 + 36)[0]
            assert elapsed >= 0
        # the largest request takes well over a microsecond of GPU time
        assert struct.unpack_from("<i", h.request_data(done, offs, 0), 4 + 36)[0] >= 1
    assert lib.destroy_htp_message_channel() == 0
    lib.close_dsp_session()
    chan.free()
    for trio in bufs:
        for b in trio:
            b.free()
