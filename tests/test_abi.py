"""Wire ABI and exported C symbols (CPU only).

- include/htp_ops/{message,op_reg}.h against the reference's own headers,
  compiled where they lie into oracle/_ref/libref_abi.so (oracle/Makefile `ref`).
- Every function declared in include/htp_ops/*.h is exported by libhtp_ops.so.
"""
import ctypes
import os
import re
import struct
import subprocess

import numpy as np
import pytest

from conftest import REPO, PKG

INCLUDE = os.path.join(REPO, "include", "htp_ops")


@pytest.fixture(scope="module")
def own(tmp_path_factory):
    out = tmp_path_factory.mktemp("abi") / "libown_abi.so"
    subprocess.run(["gcc", "-std=gnu11", "-O1", "-fPIC", "-shared", "-I", os.path.join(REPO, "include"), "-o",
                    str(out), os.path.join(REPO, "tests", "abi_probe.c")], check=True)
    lib = ctypes.CDLL(str(out))
    lib.own_abi_size.restype = ctypes.c_size_t
    lib.own_abi_size.argtypes = [ctypes.c_int]
    lib.own_abi_offset.restype = ctypes.c_size_t
    lib.own_abi_offset.argtypes = [ctypes.c_int]
    lib.own_opcode.argtypes = [ctypes.c_int]
    lib.own_message_header_validate_layout.argtypes = [ctypes.c_void_p, ctypes.c_size_t,
                                                       ctypes.POINTER(ctypes.c_size_t)]
    return lib


@pytest.fixture(scope="module")
def ref(orc):
    lib = orc.ref_lib()
    if lib is None:
        pytest.skip("oracle/_ref/libref_abi.so not built (reference sources absent)")
    return lib


EXPECTED_SIZES = {0: 16, 1: 8, 2: 4, 3: 8, 4: 128, 5: 40, 6: 64, 7: 104, 8: 17536, 9: 48, 10: 92, 11: 56,
                  12: 8, 13: 32, 14: 24, 15: 16, 16: 76, 17: 84, 18: 128, 19: 100, 20: 144}


def test_sizes_match_reference(own, ref):
    for which, size in EXPECTED_SIZES.items():
        assert own.own_abi_size(which) == ref.ref_abi_size(which) == size, which


def test_offsets_match_reference(own, ref):
    for which in range(25):
        assert own.own_abi_offset(which) == ref.ref_abi_offset(which), which


def test_opcodes_match_reference(own, ref):
    for which in range(11):
        assert own.own_opcode(which) == ref.ref_opcode(which), which
    assert own.own_opcode(1) == 15 and own.own_opcode(2) == 16 and own.own_opcode(0) == 1
    assert own.own_opcode(6) == 19
    assert [own.own_opcode(w) for w in (7, 8, 9, 10)] == [8, 10, 11, 12]


def test_packed_shape_rule_matches_reference(own, ref):
    """The head-count / head-dim rule of the QKV opcodes (reference
    include/op_reg.h:23-39) over a grid around every supported value."""
    accepted = []
    for n_heads in range(-1, 41):
        for head_dim in (-64, 0, 32, 63, 64, 65, 96, 128, 129, 256):
            for kv in (n_heads, 1, 2, 0):
                for eq in (0, 1):
                    a = own.own_packed_shape_supported(n_heads, kv, head_dim, eq)
                    assert a == ref.ref_packed_shape_supported(n_heads, kv, head_dim, eq), (n_heads, kv, head_dim, eq)
                    if a and eq:
                        accepted.append((n_heads, head_dim))
    assert sorted(set(accepted)) == [(24, 64), (24, 128), (30, 64), (30, 128), (38, 64)]


def _validate(lib, fn, raw, capacity):
    buf = (ctypes.c_uint8 * len(raw)).from_buffer_copy(raw)
    total = ctypes.c_size_t(0)
    ok = fn(ctypes.addressof(buf), capacity, ctypes.byref(total))
    return ok, total.value if ok else None


def test_layout_validation_matches_reference(own, ref):
    """The reference's own cases (op_tests.cc:606-649) plus a randomized sweep."""
    cap = 128

    def valid():
        raw = bytearray(cap)
        struct.pack_into("<i", raw, 12, 2)
        h = 16 + 4 * 3
        struct.pack_into("<3i", raw, 16, h, h + 8, h + 16)
        return raw

    cases = [valid()]
    for mutate in (lambda r: struct.pack_into("<i", r, 12, -1), lambda r: struct.pack_into("<i", r, 12, 2**31 - 1),
                   lambda r: struct.pack_into("<i", r, 16, 27), lambda r: struct.pack_into("<i", r, 20, 27),
                   lambda r: struct.pack_into("<i", r, 20, 35), lambda r: struct.pack_into("<i", r, 24, cap + 1)):
        r = valid()
        mutate(r)
        cases.append(r)
    rng = np.random.default_rng(0)
    for _ in range(4000):
        n = int(rng.integers(-2, 8))
        raw = bytearray(cap)
        struct.pack_into("<i", raw, 12, n)
        cur = int(rng.integers(0, 64))
        for i in range(max(0, min(n + 1, 28))):
            struct.pack_into("<i", raw, 16 + 4 * i, cur)
            cur += int(rng.integers(-4, 24))
        cases.append(raw)
    for raw in cases:
        for capacity in (cap, 64, 20):
            assert _validate(own, own.own_message_header_validate_layout, raw, capacity) == \
                _validate(ref, ref.ref_message_header_validate_layout, raw, capacity)


def declared_functions():
    names = set()
    for fname in os.listdir(INCLUDE):
        if not fname.endswith(".h"):
            continue  # include-path shims under host/ only forward
        text = open(os.path.join(INCLUDE, fname)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\([^;{]*\)\s*;", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    import htp_ops

    names = declared_functions()
    assert len(names) > 90
    out = subprocess.run(["nm", "-D", "--defined-only", htp_ops.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing


def test_library_loads_and_binds_every_declared_symbol():
    import htp_ops

    lib = htp_ops.lib()
    bound = set(htp_ops._SIGNATURES) | set(htp_ops._HOST_SIGNATURES)
    for name in declared_functions():
        assert getattr(lib, name) is not None
        assert name in bound, f"{name} has no Python binding"


def test_capability_markers():
    import htp_ops

    lib = htp_ops.lib()
    assert lib.htp_ops_f16_epilogue_version() == 1
    assert lib.htp_ops_native_model_version() == 0
    assert lib.htp_ops_dit_aux_version() == 1      # opcode 19 modes 9-13 are implemented
    assert lib.htp_ops_dit_concat_version() == 1


def test_wire_helpers_sizes():
    import htp_ops as h

    assert len(h.w8a8_params((1, 0), (2, 0), (3, 0), 1, 32, 64)) == 40
    assert len(h.w8a8_params((1, 0), (2, 0), (3, 0), 1, 32, 64) + h.w8a8_profile(1)) == 104
    assert len(h.f16_epilogue_params((1, 0), (2, 0), (3, 0), (-1, 0), 1, 32, 32, 32, 0)) == 56
    assert len(h.matmul_params((1, 0), (2, 0), (3, 0), 1, 32, 32)) == 92
    assert len(h.matmul_params((1, 0), (2, 0), (3, 0), 1, 32, 32, True)) == 96


def test_reference_style_caller_compiles_and_links(tmp_path):
    """tests/dropin_caller.c keeps the reference host's include lines
    ("host/session.h", <remote.h>, <rpcmem.h>, "htp_ops.h", "message.h",
    "op_reg.h"); with -I include/htp_ops it builds against libhtp_ops.so alone."""
    exe = tmp_path / "dropin"
    subprocess.run(["gcc", "-std=gnu11", "-Wall", "-Werror", "-I", INCLUDE, os.path.join(REPO, "tests", "dropin_caller.c"),
                    "-L", PKG, "-lhtp_ops", f"-Wl,-rpath,{PKG}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["40", "56", "15", "1"]
