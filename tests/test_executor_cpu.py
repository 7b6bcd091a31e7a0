"""Executor, mailbox channel and session state machine on the host (no GPU).

Every request here fails validation before any GPU work, so the return codes
of the reference dispatcher (reference src/dsp/op_executor.cc:314-540) and the
channel protocol (reference src/dsp/commu.c:99-268) are checked on the CPU.
"""
import ctypes
import struct
import time

import numpy as np
import pytest

import htp_ops as h


@pytest.fixture(scope="module")
def bufs():
    big = h.RpcBuffer(1 << 20)
    small = h.RpcBuffer(4096)
    unmapped = h.RpcBuffer(4096, map_it=False)
    yield big, small, unmapped
    for b in (big, small, unmapped):
        b.free()


def w8a8_blob(k, n):
    w = np.zeros((n, k), np.int8)
    return h.pack_constants(w, np.ones(n, np.float32))


@pytest.mark.parametrize("size", [0, 4, 39, 41, 47, 49, 103, 105])
def test_w8a8_payload_size(size):
    payload = h.w8a8_params((1, 0), (1, 0), (1, 0), 1, 32, 64) + bytes(200)
    assert h.execute(15, payload[:size])[0] == -1


@pytest.mark.parametrize("m,k,n", [(0, 32, 64), (-1, 32, 64), (65537, 32, 64), (1, 16, 64), (1, 48, 64),
                                   (1, 32800, 64), (1, 32, 32), (1, 32, 96), (1, 32, 65600)])
def test_w8a8_envelope(bufs, m, k, n):
    big = bufs[0]
    rc, _ = h.execute(15, h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 0), m, k, n))
    assert rc == -1


def test_w8a8_envelope_extension_accepts_large_k(bufs):
    """k = 14336 > 6144 (reference limit) passes validation; it fails later on
    the (deliberately bad) header with -3, not with -1."""
    big = bufs[0]
    rc, _ = h.execute(15, h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 0), 1, 14336, 64))
    assert rc == -3


def test_w8a8_unmapped_and_out_of_range(bufs):
    big, small, unmapped = bufs
    m, k, n = 4, 64, 64
    ok = (big.fd, 0)
    assert h.execute(15, h.w8a8_params((unmapped.fd, 0), ok, ok, m, k, n))[0] == -2
    assert h.execute(15, h.w8a8_params(ok, (unmapped.fd, 0), ok, m, k, n))[0] == -2
    assert h.execute(15, h.w8a8_params(ok, ok, (unmapped.fd, 0), m, k, n))[0] == -2
    assert h.execute(15, h.w8a8_params(ok, ok, (999999, 0), m, k, n))[0] == -2
    # constants range past the end of the buffer
    assert h.execute(15, h.w8a8_params(ok, ok, (small.fd, 4000), m, k, n))[0] == -2
    assert h.execute(15, h.w8a8_params(ok, ok, (small.fd, -8), m, k, n))[0] == -2


def test_w8a8_header_fields(bufs):
    big = bufs[0]
    m, k, n = 2, 64, 128
    blob = w8a8_blob(k, n)
    base = 8192
    for field in range(9):
        bad = blob.copy()
        v = np.frombuffer(bad[:36].tobytes(), np.uint32).copy()
        v[field] ^= 1
        bad[:36] = np.frombuffer(v.tobytes(), np.uint8)
        big.write(bad, base)
        assert h.execute(15, h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, base), m, k, n))[0] == -3, field


@pytest.mark.parametrize("mode", [0, 4, 0xffffffff])
def test_w8a8_profile_mode(bufs, mode):
    """Profile mode outside 1..3 is rejected after the header check."""
    big = bufs[0]
    m, k, n = 2, 64, 128
    big.write(w8a8_blob(k, n), 8192)
    payload = h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 8192), m, k, n) + h.w8a8_profile(mode)
    assert h.execute(15, payload)[0] == -1


def test_w8a8_cpu_variant_row_limit(bufs):
    big = bufs[0]
    payload = h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 0), 4097, 32, 64) + struct.pack("<ii", big.fd, 0)
    assert h.execute(15, payload)[0] == -1


def test_w8a8_cpu_variant_unmapped_control(bufs):
    big, _, unmapped = bufs
    m, k, n = 2, 64, 128
    big.write(w8a8_blob(k, n), 8192)
    payload = h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 8192), m, k, n) + struct.pack("<ii", unmapped.fd, 0)
    assert h.execute(15, payload)[0] == -2


@pytest.mark.parametrize("m,k,n,channels,mode", [
    (0, 32, 32, 32, 0), (1, 0, 32, 32, 0), (1, 32, 0, 32, 0), (1, 48, 32, 32, 0), (1, 32, 48, 48, 0),
    (1, 32, 64, 0, 3), (1, 32, 64, 65, 3), (1, 32, 64, 64, 4), (1, 32, 64, 64, -1), (1, 32, 64, 32, 0),
    (1, 32, 64, 32, 1), (1, 32, 64, 32, 2)])
def test_f16_validation(bufs, m, k, n, channels, mode):
    big = bufs[0]
    p = h.f16_epilogue_params((big.fd, 0), (big.fd, 0), (big.fd, 0), (-1, 0), m, k, n, channels, mode)
    assert h.execute(16, p)[0] == -1


def test_f16_payload_size_and_mapping(bufs):
    big, _, unmapped = bufs
    p = h.f16_epilogue_params((big.fd, 0), (big.fd, 0), (big.fd, 0), (-1, 0), 4, 64, 64, 64, 0)
    assert h.execute(16, p[:55])[0] == -1
    assert h.execute(16, p + b"\0")[0] == -1
    for i in range(4):
        addrs = [(big.fd, 0)] * 3 + [(big.fd, 0)]
        addrs[i] = (unmapped.fd, 0)
        p = h.f16_epilogue_params(*addrs, 4, 64, 64, 64, 0)
        assert h.execute(16, p)[0] == -1, i


def test_f16_alignment(bufs):
    """dst / activation / weight must be 128-byte aligned (mat_mul.c:947-949)."""
    big = bufs[0]
    for i in range(3):
        addrs = [(big.fd, 0), (big.fd, 4096), (big.fd, 65536)]
        addrs[i] = (big.fd, addrs[i][1] + 64)
        p = h.f16_epilogue_params(*addrs, (-1, 0), 4, 64, 64, 64, 0)
        assert h.execute(16, p)[0] == -12, i


def test_matmul_codes(bufs):
    big, _, unmapped = bufs
    ok = [(big.fd, 0), (big.fd, 4096), (big.fd, 65536)]
    assert h.execute(1, h.matmul_params(*ok, 4, 64, 64)[:91])[0] == -1
    for i in range(3):
        a = list(ok)
        a[i] = (unmapped.fd, 0)
        assert h.execute(1, h.matmul_params(*a, 4, 64, 64))[0] == -2
        a = list(ok)
        a[i] = (big.fd, a[i][1] + 4)
        assert h.execute(1, h.matmul_params(*a, 4, 64, 64))[0] == -3
    assert h.execute(1, h.matmul_params(*ok, 0, 64, 64))[0] == -10
    assert h.execute(1, h.matmul_params(*ok, 4, 0, 64))[0] == -10
    assert h.execute(1, h.matmul_params(*ok, -4, 64, 64))[0] == -11
    assert h.execute(1, h.matmul_params(*ok, 4, 48, 64))[0] == -11
    assert h.execute(1, h.matmul_params(*ok, 4, 64, 48))[0] == -11


@pytest.mark.parametrize("op", [0, 5, 9, 14, 17, 18, 20, 1000])
def test_unsupported_opcodes(op):
    assert h.execute(op, bytes(64))[0] == h.E_UNSUPPORTED


def test_short_request():
    buf = (ctypes.c_uint8 * 4)()
    assert h.lib().execute_op_simple(ctypes.addressof(buf), 3) == -1
    assert h.lib().execute_op_simple(None, 8) == -1


def test_canary_untouched_by_rejected_requests(bufs):
    big = bufs[0]
    for op, payload in [(15, h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 0), 0, 32, 64)),
                        (16, h.f16_epilogue_params((big.fd, 0), (big.fd, 0), (big.fd, 0), (-1, 0), 0, 32, 32, 32, 0))]:
        req = bytearray(h.compute_request(op, payload) + b"\xa5" * 64)
        buf = (ctypes.c_uint8 * len(req)).from_buffer(req)
        assert h.lib().execute_op_simple(ctypes.addressof(buf), len(req) - 64) == -1
        assert bytes(req[-64:]) == b"\xa5" * 64


# ------------------------------------------------------------- mailbox -------

def run_message(msg_buf, requests, capacity, timeout=10.0):
    msg, offsets = h.build_message(requests, capacity)
    view = msg_buf.host_view()
    view[8:len(msg)] = np.frombuffer(bytes(msg[8:]), np.uint8)
    view[:8] = 0
    view[0] = 1  # post: v[0] = 1
    t0 = time.time()
    while view[1] != 1:
        assert time.time() - t0 < timeout, "channel did not complete"
        time.sleep(0.0005)
    done = bytearray(view[:capacity].tobytes())
    return done, offsets


def test_message_layout_helpers_valid():
    msg, offsets = h.build_message([(h.REQUEST_TYPE_NO_OP, b""), (h.REQUEST_TYPE_NO_OP, b"abc")], 256)
    buf = (ctypes.c_uint8 * len(msg)).from_buffer(msg)
    assert h.lib().htp_ops_execute_message(ctypes.addressof(buf), 256) == 0
    assert h.lib().htp_ops_execute_message(ctypes.addressof(buf), 30) == -1


@pytest.fixture()
def mapping_channel():
    handle = ctypes.c_uint64()
    assert h.lib().htp_ops_open(b"", ctypes.byref(handle)) == 0
    assert h.lib().htp_ops_init_mapping_backend(handle) == 0
    chan = h.RpcBuffer(8192)
    assert h.lib().htp_ops_create_channel(handle, chan.fd, 8192) == 0
    yield handle, chan
    assert h.lib().htp_ops_destroy_channel(handle) == 0
    assert h.lib().htp_ops_close(handle) == 0
    chan.free()


def test_channel_mapping_only_compute_is_badstate(mapping_channel, bufs):
    _, chan = mapping_channel
    big = bufs[0]
    compute = h.compute_request(15, h.w8a8_params((big.fd, 0), (big.fd, 0), (big.fd, 0), 1, 32, 64))
    done, offs = run_message(chan, [(h.REQUEST_TYPE_OP_COMPUTE, compute)], 8192)
    assert h.request_state(done, offs, 0) == h.AEE_EBADSTATE
    assert done[1] == 1 and done[0] == 1


def test_channel_map_requests(mapping_channel, bufs):
    _, chan = mapping_channel
    big, small, unmapped = bufs
    v1 = struct.pack("<ii", 2, 0) + struct.pack("<ii", big.fd, 12345)
    v1_bad = struct.pack("<ii", 3, 0) + struct.pack("<ii", big.fd, small.fd)   # more puts than fds listed
    entry = lambda fd, off, size: struct.pack("<iIQQQ", fd, 0, off, size, 0)
    v2 = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 1, 1) + entry(small.fd, 0, 4096) + entry(big.fd, 0, 4096)
    v2_token = struct.pack("<IHHQii", 0x32504d52, 2, 24, 7, 0, 1) + entry(big.fd, 0, 64)
    v2_get_bad = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 0, 1) + entry(unmapped.fd, 0, 64)
    v2_put_bad = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 1, 0) + entry(424242, 0, 64)
    v2_short = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 0, 2) + entry(big.fd, 0, 64)
    done, offs = run_message(chan, [(h.REQUEST_TYPE_RPCMEM_MAP, v1), (h.REQUEST_TYPE_RPCMEM_MAP, v1_bad),
                                    (h.REQUEST_TYPE_RPCMEM_MAP, v2), (h.REQUEST_TYPE_RPCMEM_MAP, v2_token),
                                    (h.REQUEST_TYPE_RPCMEM_MAP, v2_get_bad), (h.REQUEST_TYPE_RPCMEM_MAP, v2_put_bad),
                                    (h.REQUEST_TYPE_RPCMEM_MAP, v2_short), (h.REQUEST_TYPE_RPCMEM_MAP, b"\0" * 4),
                                    (h.REQUEST_TYPE_NO_OP, b"")], 8192)
    assert [h.request_state(done, offs, i) for i in range(9)] == [0, -1, 0, -1, -1, -1, -1, -1, 0]


def test_channel_invalid_layout_completes(mapping_channel):
    _, chan = mapping_channel
    view = chan.host_view()
    view[:64] = 0
    struct.pack_into("<i", view, 12, 3)
    struct.pack_into("<4i", view, 16, 10, 50, 40, 60)  # first offset inside the table, then decreasing
    snapshot = view[16:64].copy()
    view[0] = 1
    t0 = time.time()
    while view[1] != 1:
        assert time.time() - t0 < 10
        time.sleep(0.0005)
    assert np.array_equal(view[16:64], snapshot)


def test_channel_repeated_messages(mapping_channel):
    _, chan = mapping_channel
    for i in range(20):
        done, offs = run_message(chan, [(h.REQUEST_TYPE_NO_OP, bytes(i))], 8192)
        assert done[1] == 1


# ----------------------------------------------------------- lifecycle ---------

def test_backend_state_machine_without_gpu():
    lib = h.lib()
    handle = ctypes.c_uint64()
    assert lib.htp_ops_open(b"", ctypes.byref(handle)) == 0
    chan = h.RpcBuffer(4096)
    assert lib.htp_ops_create_channel(handle, chan.fd, 4096) == h.AEE_EBADSTATE  # not initialized
    assert lib.htp_ops_init_backend_fraction(handle, 0, 1) == h.AEE_EBADPARM
    assert lib.htp_ops_init_backend_fraction(handle, 2, 1) == h.AEE_EBADPARM
    if h.device_count() == 0:
        assert lib.htp_ops_init_backend(handle) == h.AEE_EFAILED
    assert lib.htp_ops_init_mapping_backend(handle) == 0
    assert lib.htp_ops_create_channel(handle, 999999, 4096) == -1
    assert lib.htp_ops_create_channel(handle, chan.fd, 8192) == -1  # larger than the buffer
    assert lib.htp_ops_create_channel(handle, chan.fd, 4096) == 0
    assert lib.htp_ops_create_channel(handle, chan.fd, 4096) == h.AEE_EALREADY
    assert lib.htp_ops_release_backend(handle) == 0
    assert lib.htp_ops_destroy_channel(handle) == 0
    assert lib.htp_ops_destroy_channel(handle) == 0
    scope = ctypes.c_int32(0)
    assert lib.htp_ops_test_ops(handle, ctypes.byref(scope)) == h.AEE_EBADSTATE
    assert lib.htp_ops_rms_norm_f32(handle, 0, 0, 0, 0, 1, 1) == h.AEE_EBADSTATE
    assert lib.htp_ops_close(handle) == 0
    assert lib.htp_ops_close(handle) == h.AEE_EBADSTATE
    assert lib.htp_ops_init_backend(handle) == h.AEE_EBADSTATE
    chan.free()


def test_test_ops_self_checks():
    lib = h.lib()
    handle = ctypes.c_uint64()
    assert lib.htp_ops_open(b"", ctypes.byref(handle)) == 0
    assert lib.htp_ops_init_mapping_backend(handle) == 0
    scope = ctypes.c_int32(0)
    assert lib.htp_ops_test_ops(handle, None) == h.AEE_EBADPARM
    assert lib.htp_ops_test_ops(handle, ctypes.byref(scope)) == 0
    assert scope.value == 1
    assert lib.htp_ops_rms_norm_f32(handle, 0, 0, 0, 0, 1, 1) == h.AEE_EUNSUPPORTED
    assert lib.htp_ops_close(handle) == 0


def test_sessions(monkeypatch):
    lib = h.lib()
    monkeypatch.setenv("SD_HTP_MULTI_SESSION", "1")
    assert lib.open_dsp_session(3, 1) == 0
    default = lib.htp_ops_default_session()
    assert default
    assert lib.get_global_handle() == lib.htp_ops_session_handle(default)
    reserved = ctypes.c_void_p()
    assert lib.htp_ops_session_open(ctypes.byref(reserved), 3, b"x", 1) == 0
    assert lib.htp_ops_session_is_reserved(reserved) == 1
    assert lib.htp_ops_session_id(reserved) >= 1
    assert lib.htp_ops_session_domain(reserved) == 3
    assert lib.htp_ops_session_init_backend(reserved) == 0   # mapping backend under SD_HTP_MULTI_SESSION
    assert lib.htp_ops_session_is_initialized(reserved) == 1
    chan = h.RpcBuffer(4096)
    assert lib.htp_ops_session_create_channel_with_token(reserved, chan.fd, 4096) == 0
    assert lib.htp_ops_session_has_channel(reserved) == 1
    # the V2 token of a reserved session is (index << 32) | domain
    token = (lib.htp_ops_session_id(reserved) << 32) | 3
    entry = struct.pack("<iIQQQ", chan.fd, 0, 0, 64, 0)
    good = struct.pack("<IHHQii", 0x32504d52, 2, 24, token, 0, 1) + entry
    bad = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 0, 1) + entry
    # the channel buffer itself is the mailbox: use a second buffer for the message test
    assert lib.htp_ops_set_active_session(reserved) == 0
    assert lib.get_global_handle() == lib.htp_ops_session_handle(reserved)
    assert lib.htp_ops_set_default_session() == 0
    assert lib.get_global_handle() == lib.htp_ops_session_handle(default)
    assert lib.htp_ops_session_release_backend(reserved) == 0
    assert lib.htp_ops_session_is_initialized(reserved) == 0
    assert lib.htp_ops_session_destroy_channel(reserved) == 0
    lib.htp_ops_session_close(reserved)
    lib.close_dsp_session()
    assert lib.htp_ops_default_session() is None
    assert lib.htp_ops_set_default_session() == -1
    assert lib.htp_ops_session_init_backend(None) == -1
    chan.free()
    del good, bad


def test_session_token_checked_by_channel(monkeypatch):
    lib = h.lib()
    reserved = ctypes.c_void_p()
    assert lib.htp_ops_session_open(ctypes.byref(reserved), 3, b"x", 1) == 0
    handle = lib.htp_ops_session_handle(reserved)
    assert lib.htp_ops_init_mapping_backend(handle) == 0
    chan = h.RpcBuffer(4096)
    target = h.RpcBuffer(4096)
    assert lib.htp_ops_session_create_channel_with_token(reserved, chan.fd, 4096) == 0
    token = (lib.htp_ops_session_id(reserved) << 32) | 3
    entry = struct.pack("<iIQQQ", target.fd, 0, 0, 64, 0)
    good = struct.pack("<IHHQii", 0x32504d52, 2, 24, token, 0, 1) + entry
    bad = struct.pack("<IHHQii", 0x32504d52, 2, 24, 0, 0, 1) + entry
    done, offs = run_message(chan, [(h.REQUEST_TYPE_RPCMEM_MAP, good), (h.REQUEST_TYPE_RPCMEM_MAP, bad)], 4096)
    assert h.request_state(done, offs, 0) == 0 and h.request_state(done, offs, 1) == -1
    lib.htp_ops_session_close(reserved)
    chan.free()
    target.free()


def test_rpcmem_registry():
    lib = h.lib()
    assert lib.rpcmem_alloc(25, 0, 0) is None
    assert lib.rpcmem_alloc(25, 0, -5) is None
    b = h.RpcBuffer(1000, map_it=False)
    assert lib.htp_ops_amd_buffer_size(b.fd) == 1000
    assert lib.htp_ops_amd_buffer_is_device(b.fd) == 0
    assert lib.fastrpc_mmap(3, b.fd, b.ptr, 0, 2000, 2) != 0
    assert lib.fastrpc_mmap(3, 77777, None, 0, 10, 2) != 0
    assert lib.fastrpc_mmap(3, b.fd, b.ptr, 0, 1000, 2) == 0
    data = np.arange(250, dtype=np.int32)
    b.write(data)
    assert np.array_equal(b.read(np.int32, 250), data)
    with pytest.raises(h.HtpOpsError):
        b.write(data, offset=8)
    assert lib.rpcmem_to_fd(None) == -1
    assert lib.fastrpc_munmap(3, b.fd, b.ptr, 1000) == 0
    fd = b.fd
    b.free()
    assert lib.htp_ops_amd_buffer_size(fd) == -1
    assert lib.rpcmem_to_fd(ctypes.c_void_p(12345)) == -1
