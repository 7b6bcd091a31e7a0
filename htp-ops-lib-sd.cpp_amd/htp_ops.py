"""ctypes bindings of libhtp_ops.so (the C ABI declared in include/htp_ops/*.h).

Tests, the smoke check and bench.py drive the library through these bindings:
the hb_* kernel layer (device buffers, W8A8 / F16 kernels), the executor
(execute_op_simple, mailbox messages), the session / channel API and the
rpcmem buffer registry.  Nothing here computes: a missing or unloadable
library raises immediately.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhtp_ops.so")

HB_OK = 0
HB_E_HIP = -5
HB_E_NOMEM = -12
HB_E_NODEV = -19
HB_E_INVAL = -22

EPI_SCALE = 0
EPI_SCALE_GELU = 1
EPI_RAW = 2

SECTION_WEIGHTS, SECTION_SW, SECTION_DELTA, SECTION_WSUM128, SECTION_INV = range(5)

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_size_t = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    # hb runtime
    "hb_device_count": (_c_int, []),
    "hb_init": (_c_int, [_c_int]),
    "hb_last_error": (ctypes.c_char_p, []),
    "hb_default_stream": (_c_void_p, []),
    "hb_malloc": (_c_int, [ctypes.POINTER(_c_void_p), _c_size_t]),
    "hb_free": (_c_int, [_c_void_p]),
    "hb_host_malloc": (_c_int, [ctypes.POINTER(_c_void_p), _c_size_t]),
    "hb_host_free": (_c_int, [_c_void_p]),
    "hb_memcpy_h2d": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "hb_memcpy_d2h": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "hb_memcpy_d2h_async": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "hb_memcpy_d2d": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "hb_memset": (_c_int, [_c_void_p, _c_int, _c_size_t, _c_void_p]),
    "hb_stream_create": (_c_int, [ctypes.POINTER(_c_void_p)]),
    "hb_stream_destroy": (_c_int, [_c_void_p]),
    "hb_stream_sync": (_c_int, [_c_void_p]),
    "hb_device_sync": (_c_int, []),
    "hb_event_create": (_c_int, [ctypes.POINTER(_c_void_p)]),
    "hb_event_destroy": (_c_int, [_c_void_p]),
    "hb_event_record": (_c_int, [_c_void_p, _c_void_p]),
    "hb_event_sync": (_c_int, [_c_void_p]),
    "hb_event_elapsed_ms": (_c_int, [ctypes.POINTER(ctypes.c_float), _c_void_p, _c_void_p]),
    "hb_graph_begin": (_c_int, [_c_void_p]),
    "hb_graph_end": (_c_int, [ctypes.POINTER(_c_void_p), _c_void_p]),
    "hb_graph_launch": (_c_int, [_c_void_p, _c_void_p]),
    "hb_graph_destroy": (_c_int, [_c_void_p]),
    # W8A8
    "hb_w8a8_packed_bytes": (_c_size_t, [_c_int, _c_int]),
    "hb_w8a8_packed_offset": (_c_size_t, [_c_int, _c_int, _c_int]),
    "hb_w8a8_prepack": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "hb_w8a8_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "hb_w8a8_linear_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int]),
    "hb_w8a8_quantize": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "hb_w8a8_gemm": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
                              _c_int, _c_void_p]),
    "hb_w8a8_linear": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p,
                                _c_size_t, _c_void_p]),
    "hb_w8a8_planes_from_raw": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "hb_w8a8_readout": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                 _c_void_p]),
    "hb_w8a8_static_setup": (_c_int, [_c_int]),
    "hb_w8a8_linear_noalloc": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "hb_w8a8_force_tile": (_c_int, [_c_int]),
    "hb_f16_force_stream": (_c_int, [_c_int]),
    "hb_f16_force_xstream": (_c_int, [_c_int]),
    "hb_f16_force_splitk": (_c_int, [_c_int]),
    "hb_w8a8_gemm_choice": (_c_int, [_c_int, _c_int, _c_int]),
    "hb_w8a8_gemm_tile": (_c_int, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    # F16
    "hb_f16_packed_bytes": (_c_size_t, [_c_int, _c_int]),
    "hb_qk0_block_bytes": (_c_size_t, [_c_int]),
    "hb_qk0_weight_bytes": (_c_size_t, [_c_int, _c_int, _c_int]),
    "hb_qk0_prepack": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_void_p]),
    "hb_qk0_gemm_ws": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p,
                                _c_size_t, _c_void_p]),
    "hb_f16_prepack": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "hb_f16_gemm": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,
                             _c_void_p]),
    "hb_f16_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int]),
    "hb_f16_gemm_ws": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,
                                _c_void_p, _c_size_t, _c_void_p]),
    "hb_model_aux": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_c_int] * 9 + [ctypes.c_float,
                                                                                         _c_void_p]),
    "hb_model_aux_workspace_bytes": (_c_size_t, [_c_int] * 5),
    "hb_qkv_post": (_c_int, [_c_void_p] * 8 + [_c_int] * 7 + [_c_void_p]),
    "hb_qkv_gemm_workspace_bytes": (_c_size_t, [_c_int, _c_int]),
    "hb_qkv_gemm": (_c_int, [_c_void_p] * 9 + [_c_int] * 8 + [_c_void_p, _c_size_t, _c_void_p]),
    "hb_model_aux_ws": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p] + [_c_int] * 9 +
                        [ctypes.c_float, _c_void_p, _c_size_t, _c_void_p]),
}

# Host-library symbols (session, executor, registry); bound when present.
_HOST_SIGNATURES = {
    "execute_op_simple": (_c_int, [_c_void_p, _c_size_t]),
    "htp_ops_execute_message": (_c_int, [_c_void_p, _c_size_t]),
    "rpcmem_init": (None, []),
    "rpcmem_deinit": (None, []),
    "rpcmem_alloc": (_c_void_p, [_c_int, ctypes.c_uint32, _c_int]),
    "rpcmem_alloc2": (_c_void_p, [_c_int, ctypes.c_uint32, _c_size_t]),
    "rpcmem_free": (None, [_c_void_p]),
    "rpcmem_to_fd": (_c_int, [_c_void_p]),
    "fastrpc_mmap": (_c_int, [_c_int, _c_int, _c_void_p, _c_int, _c_size_t, _c_int]),
    "fastrpc_munmap": (_c_int, [_c_int, _c_int, _c_void_p, _c_size_t]),
    "htp_ops_amd_buffer_size": (ctypes.c_int64, [_c_int]),
    "htp_ops_amd_buffer_is_device": (_c_int, [_c_int]),
    "htp_ops_amd_buffer_device_ptr": (_c_void_p, [_c_int]),
    "htp_ops_amd_buffer_write": (_c_int, [_c_int, _c_size_t, _c_void_p, _c_size_t]),
    "htp_ops_amd_buffer_read": (_c_int, [_c_int, _c_size_t, _c_void_p, _c_size_t]),
    "htp_ops_amd_invalidate_weights": (_c_int, [_c_int]),
    "htp_ops_open": (_c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "htp_ops_close": (_c_int, [ctypes.c_uint64]),
    "htp_ops_init_backend": (_c_int, [ctypes.c_uint64]),
    "htp_ops_init_backend_fraction": (_c_int, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32]),
    "htp_ops_init_mapping_backend": (_c_int, [ctypes.c_uint64]),
    "htp_ops_release_backend": (_c_int, [ctypes.c_uint64]),
    "htp_ops_create_channel": (_c_int, [ctypes.c_uint64, ctypes.c_int32, ctypes.c_uint32]),
    "htp_ops_create_channel_with_token": (_c_int, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32,
                                                   ctypes.c_uint32]),
    "htp_ops_destroy_channel": (_c_int, [ctypes.c_uint64]),
    "htp_ops_rms_norm_f32": (_c_int, [ctypes.c_uint64] + [ctypes.c_int32] * 6),
    "htp_ops_mat_mul_permuted_w16a32": (_c_int, [ctypes.c_uint64] + [ctypes.c_int32] * 9),
    "htp_ops_mat_mul_permuted_w16a32_trace": (_c_int, [ctypes.c_uint64] + [ctypes.c_int32] * 9 +
                                              [ctypes.POINTER(ctypes.c_uint64)] * 3),
    "htp_ops_test_ops": (_c_int, [ctypes.c_uint64, ctypes.POINTER(ctypes.c_int32)]),
    "htp_ops_session_open": (_c_int, [ctypes.POINTER(_c_void_p), _c_int, ctypes.c_char_p, _c_int]),
    "htp_ops_default_session": (_c_void_p, []),
    "htp_ops_session_init_backend": (_c_int, [_c_void_p]),
    "htp_ops_session_acquire_backend": (_c_int, [_c_void_p]),
    "htp_ops_session_release_backend": (_c_int, [_c_void_p]),
    "htp_ops_session_create_channel": (_c_int, [_c_void_p, _c_int, ctypes.c_uint]),
    "htp_ops_session_create_channel_with_token": (_c_int, [_c_void_p, _c_int, ctypes.c_uint]),
    "htp_ops_session_destroy_channel": (_c_int, [_c_void_p]),
    "htp_ops_session_handle": (ctypes.c_uint64, [_c_void_p]),
    "htp_ops_set_active_session": (_c_int, [_c_void_p]),
    "htp_ops_set_default_session": (_c_int, []),
    "htp_ops_session_id": (ctypes.c_uint32, [_c_void_p]),
    "htp_ops_session_domain": (ctypes.c_uint32, [_c_void_p]),
    "htp_ops_session_is_reserved": (_c_int, [_c_void_p]),
    "htp_ops_session_is_initialized": (_c_int, [_c_void_p]),
    "htp_ops_session_has_channel": (_c_int, [_c_void_p]),
    "htp_ops_session_close": (None, [_c_void_p]),
    "open_dsp_session": (_c_int, [_c_int, _c_int]),
    "close_dsp_session": (None, []),
    "get_global_handle": (ctypes.c_uint64, []),
    "init_htp_backend": (None, []),
    "release_htp_backend": (_c_int, []),
    "create_htp_message_channel": (_c_int, [_c_int, ctypes.c_uint]),
    "destroy_htp_message_channel": (_c_int, []),
    "htp_ops_rpc_rms_norm_f32": (_c_int, [_c_int] * 6),
    "htp_ops_rpc_rms_norm_f32_session": (_c_int, [_c_void_p] + [_c_int] * 6),
    "htp_ops_rpc_mat_mul_permuted_w16a32": (_c_int, [_c_int] * 9),
    "htp_ops_rpc_mat_mul_permuted_w16a32_session": (_c_int, [_c_void_p] + [_c_int] * 9),
    "htp_ops_rpc_mat_mul_permuted_w16a32_trace_session": (_c_int, [_c_void_p] + [_c_int] * 9 +
                                                          [ctypes.POINTER(ctypes.c_uint64)] * 3),
    "htp_ops_f16_epilogue_version": (_c_int, []),
    "htp_ops_native_model_version": (_c_int, []),
    "htp_ops_dit_aux_version": (_c_int, []),
    "htp_ops_dit_concat_version": (_c_int, []),
    "htp_ops_w8a8_constants_bytes": (_c_size_t, [_c_int, _c_int]),
    "htp_ops_w8a8_pack_constants": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                             _c_int, _c_int, ctypes.c_uint64]),
    "htp_ops_w8a8_quantize_weights": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int]),
    "htp_ops_w8a8_pack_f16": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_void_p, _c_int, _c_int]),
    "htp_ops_fnv1a64": (ctypes.c_uint64, [_c_void_p, _c_size_t]),
    "htp_ops_f16_permute_weights": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int]),
}

_lib = None


class HtpOpsError(RuntimeError):
    pass


def lib():
    """Loads libhtp_ops.so once; raises if it is missing (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HtpOpsError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C {HERE}")
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in list(_SIGNATURES.items()) + list(_HOST_SIGNATURES.items()):
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error():
    msg = lib().hb_last_error()
    return msg.decode() if msg else ""


def check(rc, what):
    if rc != HB_OK:
        raise HtpOpsError(f"{what} failed with {rc}: {last_error()}")


_initialized = False


def init(device=0):
    """Selects the GPU; raises HtpOpsError when no GPU is usable."""
    global _initialized
    check(lib().hb_init(device), "hb_init")
    _initialized = True


def device_count():
    return lib().hb_device_count()


def sync():
    check(lib().hb_device_sync(), "hb_device_sync")


class DeviceBuffer:
    """Owned device allocation."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().hb_malloc(ctypes.byref(p), max(self.nbytes, 1)), "hb_malloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.write(arr)
        return buf

    def write(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().hb_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, None), "hb_memcpy_h2d")

    def read(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().hb_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, None), "hb_memcpy_d2h")
        return out

    def zero(self):
        check(lib().hb_memset(self.ptr, 0, self.nbytes, None), "hb_memset")
        sync()

    def fill(self, byte):
        check(lib().hb_memset(self.ptr, byte, self.nbytes, None), "hb_memset")
        sync()

    def free(self):
        if self.ptr:
            lib().hb_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- W8A8 ------------------------------------------------------------------

def kp_of(k):
    return (k + 63) // 64 * 64


def w8a8_packed_bytes(k, n):
    return lib().hb_w8a8_packed_bytes(k, n)


def w8a8_packed_offset(k, n, section):
    return lib().hb_w8a8_packed_offset(k, n, section)


def w8a8_prepack(blob_dev, k, n):
    """blob_dev: DeviceBuffer holding the constants blob -> packed DeviceBuffer."""
    packed = DeviceBuffer(w8a8_packed_bytes(k, n))
    check(lib().hb_w8a8_prepack(packed.ptr, blob_dev.ptr, k, n, None), "hb_w8a8_prepack")
    sync()
    return packed


def w8a8_workspace_bytes(m, k):
    return lib().hb_w8a8_workspace_bytes(m, k)


def w8a8_linear_workspace_bytes(m, k, n):
    """Workspace with room for hb_w8a8_linear's split-K slices where they apply."""
    return lib().hb_w8a8_linear_workspace_bytes(m, k, n)


def w8a8_quantize(x_dev, inv_ptr, m, k):
    """Returns (q DeviceBuffer [mp][kp] int8, scales DeviceBuffer f32[mp])."""
    mp = (m + 15) // 16 * 16
    q = DeviceBuffer(mp * kp_of(k))
    s = DeviceBuffer(mp * 4)
    check(lib().hb_w8a8_quantize(q.ptr, s.ptr, x_dev.ptr, inv_ptr, m, k, None), "hb_w8a8_quantize")
    sync()
    return q, s


def w8a8_gemm(y_dev, q_dev, s_dev, packed, m, k, n, epilogue=EPI_SCALE, ldy=None, stream=None):
    check(lib().hb_w8a8_gemm(y_dev.ptr, n if ldy is None else ldy, q_dev.ptr, s_dev.ptr if s_dev else None,
                             packed.ptr, m, k, n, epilogue, stream), "hb_w8a8_gemm")


def w8a8_readout(y_dev, raw_dev, s_dev, packed, m, k, n, epilogue=EPI_SCALE, ldy=None, stream=None):
    """The GEMM epilogue as its own launch: raw int32 sums (EPI_RAW output) -> f32 values."""
    check(lib().hb_w8a8_readout(y_dev.ptr, n if ldy is None else ldy, raw_dev.ptr, s_dev.ptr, packed.ptr, m, k, n,
                                epilogue, stream), "hb_w8a8_readout")


def w8a8_linear(y_dev, x_dev, packed, m, k, n, workspace, epilogue=EPI_SCALE, stream=None):
    check(lib().hb_w8a8_linear(y_dev.ptr, x_dev.ptr, packed.ptr, m, k, n, epilogue, workspace.ptr,
                               workspace.nbytes, stream), "hb_w8a8_linear")


W8A8_TILE_SHAPES = ((128, 192), (256, 192), (128, 128), (256, 256), (64, 64))


def w8a8_force_tile(index):
    """Pins the W8A8 GEMM kernel (an index into W8A8_TILE_SHAPES for the tiled
    kernel, W8A8_STREAM_TILE or W8A8_STREAM_WIDE_TILE for the streaming kernel,
    -1 = automatic); returns the previous setting."""
    prev = lib().hb_w8a8_force_tile(index)
    if prev < -1:
        check(prev, "hb_w8a8_force_tile")
    return prev


def f16_force_stream(setting):
    """Pins the F16 large-M kernel: -1 automatic, 0 the ring kernel, 1 the
    streaming kernel; returns the previous setting."""
    prev = lib().hb_f16_force_stream(setting)
    if prev < -1:
        check(prev, "hb_f16_force_stream")
    return prev


def f16_force_xstream(setting):
    """Pins the activation-streaming F16 kernel: -1 automatic, 0 never, 1
    wherever it applies; returns the previous setting."""
    prev = lib().hb_f16_force_xstream(setting)
    if prev < -1:
        check(prev, "hb_f16_force_xstream")
    return prev


def f16_force_splitk(setting):
    """Pins the F16 split-K ring path: -1 automatic, 0 never, 1 for every
    m <= 256 with a workspace; returns the previous setting."""
    prev = lib().hb_f16_force_splitk(setting)
    if prev < -1:
        check(prev, "hb_f16_force_splitk")
    return prev


W8A8_CHOICE_DECODE, W8A8_CHOICE_DECODE_TILES, W8A8_STREAM_TILE, W8A8_STREAM_WIDE_TILE = -1, -2, 5, 6


def w8a8_gemm_kernel(m, k, n):
    """Name of the kernel hb_w8a8_gemm runs for this shape."""
    choice = lib().hb_w8a8_gemm_choice(m, k, n)
    if choice == W8A8_CHOICE_DECODE:
        return "w8a8_gemm_decode (weight streaming)"
    if choice == W8A8_CHOICE_DECODE_TILES:
        return "w8a8_gemm_decode<16,8> (per 16-row tile)"
    if choice == W8A8_STREAM_TILE:
        return "w8a8_gemm_stream<256,128>"
    if choice == W8A8_STREAM_WIDE_TILE:
        return "w8a8_gemm_stream<256,192>"
    if choice < 0:
        check(choice, "hb_w8a8_gemm_choice")
    bm, bn = W8A8_TILE_SHAPES[choice]
    return f"w8a8_gemm_tiles<{bm},{bn}>"


def w8a8_planes_from_raw(out_dev, raw_dev, m, n):
    check(lib().hb_w8a8_planes_from_raw(out_dev.ptr, raw_dev.ptr, m, n, None), "hb_w8a8_planes_from_raw")


# ---- F16 -------------------------------------------------------------------

def f16_prepack(permuted_dev, k, n):
    packed = DeviceBuffer(lib().hb_f16_packed_bytes(k, n))
    check(lib().hb_f16_prepack(packed.ptr, permuted_dev.ptr, k, n, None), "hb_f16_prepack")
    sync()
    return packed


GGML_Q4_0, GGML_Q8_0, GGML_IQ4_NL = 2, 8, 20


def qk0_weight_bytes(k, n, wtype):
    return lib().hb_qk0_weight_bytes(k, n, wtype)


def qk0_prepack(blocks_dev, k, n, wtype):
    """Quantized super-blocks (device) -> the hb_f16_prepack image (hb_qk0_prepack)."""
    packed = DeviceBuffer(lib().hb_f16_packed_bytes(k, n))
    check(lib().hb_qk0_prepack(packed.ptr, blocks_dev.ptr, k, n, wtype, None), "hb_qk0_prepack")
    return packed


def qk0_gemm(y_dev, x_dev, blocks_dev, m, k, n, wtype, workspace, stream=None):
    """hb_qk0_gemm_ws: few rows (m <= 16) straight from the super-blocks."""
    check(lib().hb_qk0_gemm_ws(y_dev.ptr, x_dev.ptr, blocks_dev.ptr, m, k, n, wtype, workspace.ptr,
                               workspace.nbytes, stream), "hb_qk0_gemm_ws")


def f16_workspace_bytes(m, k, n):
    return lib().hb_f16_workspace_bytes(m, k, n)


def f16_gemm(y_dev, x_dev, packed, bias_dev, m, k, n, channels, mode, stream=None, workspace=None):
    """hb_f16_gemm, or hb_f16_gemm_ws when a workspace buffer is given (the
    split-K path for m <= 128)."""
    if workspace is None:
        check(lib().hb_f16_gemm(y_dev.ptr, x_dev.ptr, packed.ptr, bias_dev.ptr if bias_dev else None, m, k, n,
                                channels, mode, stream), "hb_f16_gemm")
    else:
        check(lib().hb_f16_gemm_ws(y_dev.ptr, x_dev.ptr, packed.ptr, bias_dev.ptr if bias_dev else None, m, k, n,
                                   channels, mode, workspace.ptr, workspace.nbytes, stream), "hb_f16_gemm_ws")


# ---- events ----------------------------------------------------------------

class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib().hb_event_create(ctypes.byref(e)), "hb_event_create")
        self.ptr = e.value

    def record(self, stream=None):
        check(lib().hb_event_record(self.ptr, stream), "hb_event_record")

    def synchronize(self):
        check(lib().hb_event_sync(self.ptr), "hb_event_sync")

    def elapsed_ms(self, later):
        ms = ctypes.c_float()
        check(lib().hb_event_elapsed_ms(ctypes.byref(ms), self.ptr, later.ptr), "hb_event_elapsed_ms")
        return ms.value

    def __del__(self):
        try:
            lib().hb_event_destroy(self.ptr)
        except Exception:
            pass


class Graph:
    """Work captured from a stream: `with Graph.capture(stream) as g:` enqueue
    library calls on stream, then g.launch(stream) replays them."""

    def __init__(self):
        self.ptr = None

    @classmethod
    def capture(cls, stream):
        return _GraphCapture(cls(), stream)

    def launch(self, stream=None):
        if not self.ptr:
            raise HtpOpsError("graph launched after destroy()")
        check(lib().hb_graph_launch(self.ptr, stream), "hb_graph_launch")

    def destroy(self):
        """Frees the instantiated graph now (callers destroy a graph before
        freeing the buffers its launches use; __del__ is only a fallback)."""
        if self.ptr:
            ptr, self.ptr = self.ptr, None
            check(lib().hb_graph_destroy(ptr), "hb_graph_destroy")

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class _GraphCapture:
    def __init__(self, graph, stream):
        self.graph, self.stream = graph, stream

    def __enter__(self):
        check(lib().hb_graph_begin(self.stream), "hb_graph_begin")
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        g = ctypes.c_void_p()
        rc = lib().hb_graph_end(ctypes.byref(g), self.stream)
        self.graph.ptr = g.value
        if exc_type is None:
            check(rc, "hb_graph_end")
        return False


def default_stream():
    return lib().hb_default_stream()


# ---- host packers ------------------------------------------------------------

def _arr_ptr(a):
    return None if a is None else a.ctypes.data


def pack_constants(w_nk, sw, sums=None, inv=None, signature=0):
    """int8 weights [n][k] + per-column scales -> W8A8 constants blob (uint8)."""
    w_nk = np.ascontiguousarray(w_nk, np.int8)
    n, k = w_nk.shape
    nbytes = lib().htp_ops_w8a8_constants_bytes(k, n)
    blob = np.zeros(nbytes, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    sums = None if sums is None else np.ascontiguousarray(sums, np.int32)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    rc = lib().htp_ops_w8a8_pack_constants(blob.ctypes.data, nbytes, w_nk.ctypes.data, sw.ctypes.data,
                                           _arr_ptr(sums), _arr_ptr(inv), k, n, signature)
    if rc != 0:
        raise HtpOpsError(f"htp_ops_w8a8_pack_constants failed ({rc})")
    return blob


def quantize_weights(w_nk_f32, inv=None):
    w = np.ascontiguousarray(w_nk_f32, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    sw = np.empty(n, np.float32)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    rc = lib().htp_ops_w8a8_quantize_weights(q.ctypes.data, sw.ctypes.data, w.ctypes.data, _arr_ptr(inv), k, n)
    if rc != 0:
        raise HtpOpsError("htp_ops_w8a8_quantize_weights failed")
    return q, sw


def pack_f16(w_nk_f16, inv=None):
    """fp16 weights [n][k] (float16 array or uint16 bits) -> W8A8 constants blob
    (quantized per output channel, original_f16_signature = FNV-1a 64 of the fp16 bytes)."""
    w = np.ascontiguousarray(w_nk_f16).view(np.uint16)
    n, k = w.shape
    nbytes = lib().htp_ops_w8a8_constants_bytes(k, n)
    blob = np.zeros(nbytes, np.uint8)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    rc = lib().htp_ops_w8a8_pack_f16(blob.ctypes.data, blob.nbytes, w.ctypes.data, _arr_ptr(inv), k, n)
    if rc != 0:
        raise HtpOpsError("htp_ops_w8a8_pack_f16 failed")
    return blob


def permute_f16(w_kn_bits):
    w = np.ascontiguousarray(w_kn_bits, np.uint16)
    k, n = w.shape
    out = np.zeros(k * n, np.uint16)
    rc = lib().htp_ops_f16_permute_weights(out.ctypes.data, w.ctypes.data, k, n)
    if rc != 0:
        raise HtpOpsError("htp_ops_f16_permute_weights failed")
    return out


# ---- wire format ---------------------------------------------------------------

import struct as _struct

OP_MAT_MUL_PERMUTED_W16A32 = 1
OP_MAT_MUL_PERMUTED_W4D16A32 = 2
OP_MAT_MUL_PERMUTED_W8D16A32 = 3
OP_MAT_MUL_PERMUTED_W4D16A32_IQ4_NL = 4
OP_MAT_MUL_NATIVE_W8A8 = 15
OP_MAT_MUL_F16_EPILOGUE = 16
E_UNSUPPORTED = -95
REQUEST_TYPE_NO_OP, REQUEST_TYPE_RPCMEM_MAP, REQUEST_TYPE_OP_COMPUTE = 0, 1, 2
RPCMEM_FLAG_AMD_DEVICE = 1 << 30
RPCMEM_HEAP_ID_SYSTEM = 25
AEE_SUCCESS, AEE_EFAILED, AEE_ENOMEMORY, AEE_EBADSTATE, AEE_EBADPARM, AEE_EUNSUPPORTED, AEE_EALREADY = \
    0, 1, 2, 13, 14, 20, 26


def w8a8_params(out, act, cst, m, k, n, elapsed=0):
    """NativeW8A8Params (40 bytes); out/act/cst are (fd, offset)."""
    return _struct.pack("<6i4i", *out, *act, *cst, m, k, n, elapsed)


def w8a8_profile(mode):
    """NativeW8A8Profile trailer (64 bytes)."""
    return _struct.pack("<2I7Q", mode, 0, 0, 0, 0, 0, 0, 0, 0)


def unpack_w8a8_profile(raw):
    f = _struct.unpack("<2I7Q", raw)
    keys = ("mode", "reserved", "setup_ticks", "activation_ticks", "weight_ticks", "hmx_ticks", "output_ticks",
            "mac_ticks", "readout_ticks")
    return dict(zip(keys, f))


def f16_epilogue_params(out, act, wgt, bias, m, k, n, channels, mode, elapsed=0):
    """F16EpilogueParams (56 bytes)."""
    return _struct.pack("<8i6i", *out, *act, *wgt, *bias, m, k, n, channels, mode, elapsed)


def aux_params(out, inp, wgt, bias, mode, count, width, channels, spatial, groups, batch, other_count, activation,
               eps, elapsed=0):
    """NativeAuxParams (76 bytes, opcode 19); a buffer (-1, 0) is absent."""
    return _struct.pack("<8i9ifi", *out, *inp, *wgt, *bias, mode, count, width, channels, spatial, groups, batch,
                        other_count, activation, eps, elapsed)


def model_aux_workspace_bytes(mode, channels, spatial, groups, batch):
    return lib().hb_model_aux_workspace_bytes(mode, channels, spatial, groups, batch)


def model_aux(y_dev, x_dev, w_dev, b_dev, mode, count, width, channels=1, spatial=1, groups=1, batch=1,
              other_count=0, activation=0, eps=0.0, stream=None, workspace=None):
    """hb_model_aux on device buffers (w_dev / b_dev may be None), or
    hb_model_aux_ws when a workspace buffer is given."""
    w, b = (w_dev.ptr if w_dev else None), (b_dev.ptr if b_dev else None)
    if workspace is None:
        check(lib().hb_model_aux(y_dev.ptr, x_dev.ptr, w, b, mode, count, width, channels, spatial, groups, batch,
                                 other_count, activation, eps, stream), "hb_model_aux")
    else:
        check(lib().hb_model_aux_ws(y_dev.ptr, x_dev.ptr, w, b, mode, count, width, channels, spatial, groups, batch,
                                    other_count, activation, eps, workspace.ptr, workspace.nbytes, stream),
              "hb_model_aux_ws")


OP_QKV_MUL_RMS_PACKED, OP_QKV_MUL_RMS_PACKED_DUAL, OP_QKV_MUL_RMS_PACKED_ROPE, OP_QKV_MUL_RMS_PACKED_DUAL_ROPE = \
    8, 10, 11, 12
_NO_BUFFER = (-1, 0)


def qkv_params(q, k, v, act, wgt, bias, q_norm, k_norm, tokens, input_dim, n_heads, head_dim, elapsed=0):
    """QkvMulRmsPackedParams (84 bytes, opcode 8); buffers are (fd, offset)."""
    return _struct.pack("<16i5i", *q, *k, *v, *act, *wgt, *bias, *q_norm, *k_norm, tokens, input_dim, n_heads,
                        head_dim, elapsed)


def qkv_rope_params(q, k, v, act, wgt, bias, q_norm, k_norm, pe, tokens, input_dim, n_heads, head_dim,
                    rope_offset, rope_count, elapsed=0):
    """QkvMulRmsPackedRopeParams (100 bytes, opcode 11); bias may be (-1, 0)."""
    return _struct.pack("<18i7i", *q, *k, *v, *act, *wgt, *bias, *q_norm, *k_norm, *pe, tokens, input_dim, n_heads,
                        head_dim, rope_offset, rope_count, elapsed)


def qkv_dual_params(q, k, v, image, text, image_tokens, text_tokens, input_dim, n_heads, head_dim, elapsed=0):
    """QkvMulRmsPackedDualParams (128 bytes, opcode 10); image / text are
    (activation, weight, bias, q_norm, k_norm) tuples of (fd, offset)."""
    bufs = [x for b in (q, k, v, *image, *text) for x in b]
    return _struct.pack("<26i6i", *bufs, image_tokens, text_tokens, input_dim, n_heads, head_dim, elapsed)


def qkv_dual_rope_params(q, k, v, image, text, pe, image_tokens, text_tokens, input_dim, n_heads, head_dim,
                         image_rope_offset, text_rope_offset, elapsed=0):
    """QkvMulRmsPackedDualRopeParams (144 bytes, opcode 12)."""
    bufs = [x for b in (q, k, v, *image, *text, pe) for x in b]
    return _struct.pack("<28i8i", *bufs, image_tokens, text_tokens, input_dim, n_heads, head_dim, image_rope_offset,
                        text_rope_offset, elapsed)


def qkv_head_elems(token_tiles, head_dim):
    """Halfwords of one head's region in a packed Q / K / V output."""
    return token_tiles * (head_dim // 32) * 1024


def qkv_post(q_dev, k_dev, v_dev, raw_dev, bias_dev, q_norm_dev, k_norm_dev, pe_dev, rope_offset, rope_count,
             tokens, n_heads, head_dim, token_tiles, out_offset=0, stream=None):
    """hb_qkv_post on device buffers (bias_dev / pe_dev may be None)."""
    b = bias_dev.ptr if bias_dev else None
    pe = pe_dev.ptr if pe_dev else None
    check(lib().hb_qkv_post(q_dev.ptr, k_dev.ptr, v_dev.ptr, raw_dev.ptr, b, q_norm_dev.ptr, k_norm_dev.ptr, pe,
                            rope_offset, rope_count, tokens, n_heads, head_dim, token_tiles, out_offset, stream),
          "hb_qkv_post")


def qkv_gemm_workspace_bytes(tokens, input_dim):
    return lib().hb_qkv_gemm_workspace_bytes(tokens, input_dim)


def qkv_gemm(q_dev, k_dev, v_dev, x_dev, packed, bias_dev, q_norm_dev, k_norm_dev, pe_dev, rope_offset, rope_count,
             tokens, input_dim, n_heads, head_dim, token_tiles, out_offset, workspace, stream=None):
    """hb_qkv_gemm: the GEMM with the post-processing in its epilogue."""
    b = bias_dev.ptr if bias_dev else None
    pe = pe_dev.ptr if pe_dev else None
    check(lib().hb_qkv_gemm(q_dev.ptr, k_dev.ptr, v_dev.ptr, x_dev.ptr, packed.ptr, b, q_norm_dev.ptr,
                            k_norm_dev.ptr, pe, rope_offset, rope_count, tokens, input_dim, n_heads, head_dim,
                            token_tiles, out_offset, workspace.ptr, workspace.nbytes, stream), "hb_qkv_gemm")


def matmul_params(out, act, wgt, m, k, n, with_elapsed=False):
    """MatMulParams (92 bytes), optionally with the elapsed_us trailer (96)."""
    raw = _struct.pack("<6i3iQIiiQiQQQ", *out, *act, *wgt, m, k, n, 0, 0, 0, 0, 0, 0, 0, 0, 0)
    assert len(raw) == 92
    return raw + (_struct.pack("<i", 0) if with_elapsed else b"")


def compute_request(op, payload):
    """OpComputeRequest bytes: opcode + payload."""
    return _struct.pack("<I", op) + payload


def execute(op, payload):
    """Runs execute_op_simple on a copy of the request; returns (rc, payload after)."""
    req = bytearray(compute_request(op, payload))
    buf = (ctypes.c_uint8 * len(req)).from_buffer(req)
    rc = lib().execute_op_simple(ctypes.addressof(buf), len(req))
    return rc, bytes(req[4:])


def build_message(requests, capacity):
    """requests: list of (type, data bytes) -> mailbox bytes (state zeroed)."""
    n = len(requests)
    header = 16 + 4 * (n + 1)
    offsets = [header]
    for _, data in requests:
        offsets.append(offsets[-1] + 8 + len(data))
    assert offsets[-1] <= capacity
    msg = bytearray(capacity)
    _struct.pack_into("<QIi", msg, 0, 0, 0, n)
    _struct.pack_into(f"<{n + 1}i", msg, 16, *offsets)
    for i, (rtype, data) in enumerate(requests):
        _struct.pack_into("<ii", msg, offsets[i], 0, rtype)
        msg[offsets[i] + 8:offsets[i] + 8 + len(data)] = data
    return msg, offsets


def request_state(msg, offsets, i):
    return _struct.unpack_from("<i", msg, offsets[i])[0]


def request_data(msg, offsets, i):
    return bytes(msg[offsets[i] + 8:offsets[i + 1]])


class RpcBuffer:
    """An rpcmem allocation registered with the library (host or HBM)."""

    def __init__(self, nbytes, device=False, map_it=True):
        self.nbytes = int(nbytes)
        self.device = device
        flags = RPCMEM_FLAG_AMD_DEVICE if device else 0
        self.ptr = lib().rpcmem_alloc2(RPCMEM_HEAP_ID_SYSTEM, flags, self.nbytes)
        if not self.ptr:
            raise HtpOpsError("rpcmem_alloc2 failed")
        self.fd = lib().rpcmem_to_fd(self.ptr)
        if map_it:
            rc = lib().fastrpc_mmap(3, self.fd, self.ptr, 0, self.nbytes, 2)
            if rc != 0:
                raise HtpOpsError(f"fastrpc_mmap failed ({rc})")

    def write(self, arr, offset=0):
        raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
        rc = lib().htp_ops_amd_buffer_write(self.fd, offset, raw.ctypes.data, raw.nbytes)
        if rc != 0:
            raise HtpOpsError(f"htp_ops_amd_buffer_write failed ({rc})")

    def read(self, dtype, count, offset=0):
        out = np.empty(count, np.dtype(dtype))
        rc = lib().htp_ops_amd_buffer_read(self.fd, offset, out.ctypes.data, out.nbytes)
        if rc != 0:
            raise HtpOpsError(f"htp_ops_amd_buffer_read failed ({rc})")
        return out

    def host_view(self):
        """uint8 numpy view of host memory (host buffers only)."""
        assert not self.device
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(self.ptr))

    def free(self):
        if self.ptr:
            lib().rpcmem_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
