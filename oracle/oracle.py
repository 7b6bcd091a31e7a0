"""ctypes bindings of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker / CPU baseline; never by the product path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_abi.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_S = ctypes.c_size_t

_SIGS = {
    "oracle_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "oracle_f32_to_f16_array": (None, [_P, _P, _S]),
    "oracle_f16_to_f32_array": (None, [_P, _P, _S]),
    "oracle_w8a8_quantize_values": (None, [_P, _P, _S]),
    "oracle_w8a8_blob_bytes": (_S, [_I, _I]),
    "oracle_w8a8_weight_offset": (_S, [_I, _I, _I]),
    "oracle_w8a8_pack_blob": (None, [_P, _P, _P, _P, _P, _I, _I, ctypes.c_uint64]),
    "oracle_w8a8_unpack_weights": (None, [_P, _P, _I, _I]),
    "oracle_w8a8_check_header": (_I, [_P, _I, _I]),
    "oracle_w8a8_quantize_value": (ctypes.c_uint8, [ctypes.c_float]),
    "oracle_w8a8_quantize": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "oracle_w8a8_accumulate": (None, [_P, _P, _P, _I, _I, _I, _I]),
    "oracle_w8a8_output": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "oracle_w8a8_linear": (None, [_P, _P, _P, _I, _I, _I, _I]),
    "oracle_w8a8_planes": (None, [_P, _P, _I, _I]),
    "oracle_gelu_tanh": (ctypes.c_float, [ctypes.c_float]),
    "oracle_quick_gelu": (ctypes.c_float, [ctypes.c_float]),
    "oracle_gelu_tanh_inplace": (None, [_P, _S]),
    "oracle_silu": (ctypes.c_float, [ctypes.c_float]),
    "oracle_model_aux": (_I, [_P, _P, _P, _P] + [_I] * 9 + [ctypes.c_float]),
    "oracle_f16_permuted_index": (_S, [_I, _I, _I]),
    "oracle_f16_permute": (None, [_P, _P, _I, _I]),
    "oracle_f16_gemm_epilogue": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "oracle_qkv_index": (_S, [_I, _I, _I, _I, _I, _I]),
    "oracle_qkv_rsqrt": (ctypes.c_float, [ctypes.c_float]),
    "oracle_qkv_post": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]),
    "oracle_qk0_block_bytes": (_S, [_I]),
    "oracle_qk0_value": (ctypes.c_uint16, [_P, _I, _I]),
    "oracle_qk0_dequant": (_I, [_P, _P, _I, _I, _I]),
    "oracle_fill_normal": (None, [_P, _S, ctypes.c_float, ctypes.c_float, ctypes.c_uint64]),
    "oracle_fill_uniform": (None, [_P, _S, ctypes.c_float, ctypes.c_float, ctypes.c_uint64]),
    "oracle_fill_int8": (None, [_P, _S, _I, _I, ctypes.c_uint64]),
    "oracle_num_threads": (_I, []),
}

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C {HERE})")
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ref_lib():
    """The reference-header ABI probe, or None when it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = ctypes.CDLL(REF_PATH)
        _ref.ref_abi_size.restype = _S
        _ref.ref_abi_size.argtypes = [_I]
        _ref.ref_abi_offset.restype = _S
        _ref.ref_abi_offset.argtypes = [_I]
        _ref.ref_opcode.restype = _I
        _ref.ref_opcode.argtypes = [_I]
        _ref.ref_message_header_validate_layout.restype = _I
        _ref.ref_message_header_validate_layout.argtypes = [_P, _S, ctypes.POINTER(_S)]
    return _ref


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---- inputs ------------------------------------------------------------------

def normal(count, mean=0.0, std=1.0, seed=0):
    out = np.empty(count, np.float32)
    lib().oracle_fill_normal(_ptr(out), count, mean, std, seed)
    return out


def uniform(count, lo, hi, seed=0):
    out = np.empty(count, np.float32)
    lib().oracle_fill_uniform(_ptr(out), count, lo, hi, seed)
    return out


def int8_uniform(count, lo=-127, hi=127, seed=0):
    out = np.empty(count, np.int8)
    lib().oracle_fill_int8(_ptr(out), count, lo, hi, seed)
    return out


# ---- binary16 ----------------------------------------------------------------

def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(out), _ptr(x), x.size)
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().oracle_f16_to_f32_array(_ptr(out), _ptr(h), h.size)
    return out


def quantize_values(v):
    v = np.ascontiguousarray(v, np.float32).ravel()
    out = np.empty(v.size, np.uint8)
    lib().oracle_w8a8_quantize_values(_ptr(out), _ptr(v), v.size)
    return out


# ---- W8A8 --------------------------------------------------------------------

def blob_bytes(k, n):
    return lib().oracle_w8a8_blob_bytes(k, n)


def weight_offset(k, n_idx, k_idx):
    return lib().oracle_w8a8_weight_offset(k, n_idx, k_idx)


def pack_blob(w_nk, sw, sums=None, inv=None, signature=0):
    """w_nk: int8 [n][k] -> constants blob (uint8).  The weight section holds
    64-column groups of 32-row blocks, so only k % 32 == 0 and n % 64 == 0
    address inside it; other shapes are refused before the C packer runs."""
    w_nk = np.ascontiguousarray(w_nk, np.int8)
    n, k = w_nk.shape
    if k < 32 or k % 32 or n < 64 or n % 64:
        raise ValueError(f"W8A8 blob needs k % 32 == 0 and n % 64 == 0 (k={k}, n={n})")
    blob = np.zeros(blob_bytes(k, n), np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    sums = None if sums is None else np.ascontiguousarray(sums, np.int32)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    if sw.size != n or (sums is not None and sums.size != n) or (inv is not None and inv.size != k):
        raise ValueError("W8A8 blob: sw and sums need n entries, inv k entries")
    lib().oracle_w8a8_pack_blob(_ptr(blob), _ptr(w_nk), _ptr(sw), _ptr(sums), _ptr(inv), k, n, signature)
    return blob


def unpack_weights(blob, k, n):
    w = np.empty((n, k), np.int8)
    lib().oracle_w8a8_unpack_weights(_ptr(w), _ptr(np.ascontiguousarray(blob)), k, n)
    return w


def check_header(blob, k, n):
    return lib().oracle_w8a8_check_header(_ptr(np.ascontiguousarray(blob)), k, n)


def quantize_value(v):
    return lib().oracle_w8a8_quantize_value(float(v))


def quantize(x, inv, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    u = np.empty((m, k), np.uint8)
    s = np.empty(m, np.float32)
    lib().oracle_w8a8_quantize(_ptr(u), _ptr(s), _ptr(x), _ptr(np.ascontiguousarray(inv, np.float32)), m, k,
                               nthreads)
    return u, s


def accumulate(u, blob, k, n, nthreads=0):
    u = np.ascontiguousarray(u, np.uint8)
    m = u.shape[0]
    acc = np.empty((m, n), np.int32)
    lib().oracle_w8a8_accumulate(_ptr(acc), _ptr(u), _ptr(np.ascontiguousarray(blob)), m, k, n, nthreads)
    return acc


def output(acc, s, blob, k, n, nthreads=0):
    acc = np.ascontiguousarray(acc, np.int32)
    m = acc.shape[0]
    y = np.empty((m, n), np.float32)
    lib().oracle_w8a8_output(_ptr(y), _ptr(acc), _ptr(np.ascontiguousarray(s, np.float32)),
                             _ptr(np.ascontiguousarray(blob)), m, k, n, nthreads)
    return y


def linear(x, blob, k, n, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    m = x.shape[0]
    y = np.empty((m, n), np.float32)
    lib().oracle_w8a8_linear(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(blob)), m, k, n, nthreads)
    return y


def planes(acc):
    acc = np.ascontiguousarray(acc, np.int32)
    m, n = acc.shape
    out = np.zeros(m * n * 4, np.uint8)
    lib().oracle_w8a8_planes(_ptr(out), _ptr(acc), m, n)
    return out


def gelu_tanh(z):
    return lib().oracle_gelu_tanh(float(z))


def quick_gelu(z):
    return lib().oracle_quick_gelu(float(z))


def gelu_tanh_array(y):
    y = np.array(y, np.float32, copy=True)
    lib().oracle_gelu_tanh_inplace(_ptr(y), y.size)
    return y


def silu(z):
    return lib().oracle_silu(float(z))


# ---- opcode 19 ---------------------------------------------------------------

def model_aux(x, w, b, mode, count, width, channels=1, spatial=1, groups=1, batch=1, other_count=0, activation=0,
              eps=0.0, out=None):
    """Opcode-19 restatement; `out` (float32, count values) supplies the values a
    mode leaves untouched (rows past count/width), zeros when omitted."""
    x = np.ascontiguousarray(x, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    y = np.zeros(count, np.float32) if out is None else np.array(out, np.float32, copy=True)
    rc = lib().oracle_model_aux(_ptr(y), _ptr(x), _ptr(w), _ptr(b), mode, count, width, channels, spatial, groups,
                                batch, other_count, activation, float(eps))
    if rc:
        raise ValueError(f"oracle_model_aux rejected mode {mode}")
    return y


# ---- F16 ---------------------------------------------------------------------

def f16_permuted_index(k_total, k_idx, n_idx):
    return lib().oracle_f16_permuted_index(k_total, k_idx, n_idx)


def f16_permute(w_kn_bits):
    w = np.ascontiguousarray(w_kn_bits, np.uint16)
    k, n = w.shape
    out = np.zeros(k * n, np.uint16)
    lib().oracle_f16_permute(_ptr(out), _ptr(w), k, n)
    return out


def f16_gemm_epilogue(x, permuted, bias, m, k, n, channels, mode, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(m * (channels if mode == 3 else n), np.float32)
    lib().oracle_f16_gemm_epilogue(_ptr(y), _ptr(x), _ptr(np.ascontiguousarray(permuted, np.uint16)),
                                   _ptr(None if bias is None else np.ascontiguousarray(bias, np.float32)), m, k, n,
                                   channels, mode, nthreads)
    return y.reshape((channels, m) if mode == 3 else (m, n))


# ---- fused QKV + RMS + RoPE packing (opcodes 8/10/11/12) -----------------------


def qkv_index(which, token_tiles, head_dim, tt, r, c):
    return lib().oracle_qkv_index(which, token_tiles, head_dim, tt, r, c)


def qkv_rsqrt(x):
    return lib().oracle_qkv_rsqrt(x)


def qkv_head_elems(token_tiles, head_dim):
    return token_tiles * (head_dim // 32) * 1024


def qkv_post(raw, bias, q_norm, k_norm, pe, rope_offset, rope_count, tokens, n_heads, head_dim, token_tiles,
             out_offset=0, out=None):
    """Post-processing of one call's GEMM output (tokens x 3*n_heads*head_dim,
    f32 holding fp16 values) into the packed fp16 Q/K/V images (uint16 bits of
    n_heads * token_tiles * head_dim * 32 halfwords each); `out` (q, k, v)
    keeps the token tiles other calls wrote."""
    size = n_heads * qkv_head_elems(token_tiles, head_dim)
    q, k, v = out if out is not None else (np.zeros(size, np.uint16) for _ in range(3))
    raw = np.ascontiguousarray(raw, np.float32)
    f = (lambda a: None if a is None else np.ascontiguousarray(a, np.float32))
    lib().oracle_qkv_post(_ptr(q), _ptr(k), _ptr(v), _ptr(raw), _ptr(f(bias)), _ptr(f(q_norm)), _ptr(f(k_norm)),
                          _ptr(f(pe)), rope_offset, rope_count, tokens, n_heads, head_dim, token_tiles, out_offset)
    return q, k, v


# ---- dequantizing GEMM (opcodes 2/3/4) ----------------------------------------

GGML_Q4_0, GGML_Q8_0, GGML_IQ4_NL = 2, 8, 20


def qk0_block_bytes(wtype):
    return lib().oracle_qk0_block_bytes(wtype)


def qk0_value(block, j, wtype):
    return lib().oracle_qk0_value(_ptr(np.ascontiguousarray(block, np.uint8)), j, wtype)


def qk0_dequant(blocks, k, n, wtype):
    """Super-blocks (uint8) -> the permuted F16 image (uint16 bits) of opcode 1."""
    out = np.zeros(k * n, np.uint16)
    rc = lib().oracle_qk0_dequant(_ptr(out), _ptr(np.ascontiguousarray(blocks, np.uint8)), k, n, wtype)
    if rc:
        raise ValueError(f"oracle_qk0_dequant rejected k={k} n={n} type={wtype}")
    return out


def num_threads():
    return lib().oracle_num_threads()
