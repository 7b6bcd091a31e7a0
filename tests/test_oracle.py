"""Pins the CPU oracle (oracle/htp_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something it does not itself contain:
the reference's own known-answer constructions (tests/hmx-probe), the
reference's addressing formulas as written in its consumer / probe code,
closed forms and independent IEEE implementations (numpy), and brute force.
Reference citations are to files under the reference repository.
"""
import numpy as np
import pytest


# ---------------------------------------------------------------- binary16 ----

def test_f16_to_f32_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_against_numpy(orc):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # every tie and neighbour around the half grid in the normal and subnormal range
    halves = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = np.nextafter(halves, np.float32(np.inf))
    mids = ((halves.astype(np.float64) + np.roll(halves, -1).astype(np.float64)) / 2).astype(np.float32)
    extra = np.concatenate([halves, -halves, mids, -mids, nxt, np.nextafter(mids, np.float32(0)),
                            np.nextafter(mids, np.float32(np.inf)),
                            np.array([65504, 65519.99, 65520, 1e9, 2.0**-24, 2.0**-25, 2.0**-26, 3 * 2.0**-26],
                                     np.float32)])
    x = np.concatenate([x, extra])
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)


# ------------------------------------------------------------ quantization ----

def test_quantize_value_is_rint_of_clamp(orc):
    """reference linear_w8a8.c:47-58: integer clamp to [1, 255] then the
    mantissa-shift round equals IEEE round-half-even (numpy.rint)."""
    grid = np.arange(1, 256, dtype=np.float64)
    ties = (grid[:-1] + 0.5).astype(np.float32)
    rng = np.random.default_rng(1)
    dense = rng.uniform(0.5, 256.0, 2_000_000).astype(np.float32)
    v = np.concatenate([grid.astype(np.float32), ties, np.nextafter(ties, np.float32(0)),
                        np.nextafter(ties, np.float32(300)), dense])
    got = orc.quantize_values(v)
    ref = np.rint(np.clip(v, 1.0, 255.0)).astype(np.uint8)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("value,expect", [
    (-0.0, 1), (-5.0, 1), (0.0, 1), (0.25, 1), (0.999, 1), (1.5, 2), (2.5, 2), (254.5, 254), (255.49, 255),
    (300.0, 255), (float("inf"), 255), (float("-inf"), 1)])
def test_quantize_value_clamp_cases(orc, value, expect):
    assert orc.quantize_value(value) == expect


def test_quantize_value_nan_sign(orc):
    """The clamp compares IEEE bits as signed integers: +NaN -> 255, -NaN -> 1."""
    pos = np.array([0x7fc00000], np.uint32).view(np.float32)[0]
    neg = np.array([0xffc00000], np.uint32).view(np.float32)[0]
    assert orc.quantize_value(pos) == 255
    assert orc.quantize_value(neg) == 1


def test_quantize_unit_scale_row(orc):
    """max|t| = 127 gives s = 1 exactly and u = rne(t + 128) (ties to even)."""
    t = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -127.0, 3.49, -126.5] + [0.0] * 23, np.float32)
    u, s = orc.quantize(t[None, :], np.ones(32, np.float32))
    assert s[0] == np.float32(1.0)
    assert list(u[0, :9]) == [255, 128, 130, 130, 128, 126, 1, 131, 2]


def test_quantize_zero_and_tiny_rows(orc):
    """Floor s = 1e-12 (reference linear_w8a8.c:39): a zero row quantizes to 128."""
    x = np.zeros((3, 64), np.float32)
    x[1, 5] = 1e-13
    x[2, 7] = -3e-9
    u, s = orc.quantize(x, np.ones(64, np.float32))
    assert s[0] == np.float32(1e-12) and s[1] == np.float32(1e-12)
    assert (u[0] == 128).all()
    assert s[2] == np.float32(np.float32(3e-9) / np.float32(127.0))
    # 1e-13 * (1/1e-12) = 0.1 -> 128.1 -> 128; the row's maximum maps to -127 -> 1
    assert (u[1] == 128).all() and u[2, 7] == 1


def test_quantize_matches_numpy_ieee(orc):
    """Same steps in numpy float32 (one IEEE rounding per operation)."""
    rng = np.random.default_rng(2)
    m, k = 37, 320
    x = (rng.standard_normal((m, k)) * rng.uniform(1e-6, 1e3, (m, 1))).astype(np.float32)
    inv = rng.uniform(0.5, 2.0, k).astype(np.float32)
    u, s = orc.quantize(x, inv)
    t = x * inv
    amax = np.abs(t).max(axis=1)
    s_ref = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    r = (np.float32(1.0) / s_ref).astype(np.float32)
    v = (t * r[:, None]).astype(np.float32) + np.float32(128.0)
    u_ref = np.rint(np.clip(v, 1.0, 255.0)).astype(np.uint8)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(u, u_ref)


# --------------------------------------------------------------- blob layout ----

def reference_weight_offset(k, n, kk):
    """W(n,k) address composed from the reference's own expressions:
    64-column group base `n0*k` (linear_w8a8.c:453), K32 block `t*2048`
    (linear_w8a8.c:487), 32-column bank `h*1024` (study_dsp.c:82, wb=1024,
    banks=2) and the in-bank `(k/4)*128 + n*4 + k%4` (integer_tests.c:10)."""
    group = (n // 64) * 64 * k
    block = (kk // 32) * 2048
    bank = ((n % 64) // 32) * 1024
    inner = ((kk % 32) // 4) * 128 + (n % 32) * 4 + (kk % 4)
    return 128 + group + block + bank + inner


def test_weight_offset_matches_reference_formulas(orc):
    for k, n in [(32, 64), (96, 128), (1536, 192)]:
        for col in range(0, n, 7):
            for kk in range(0, k, 5):
                assert orc.weight_offset(k, col, kk) == reference_weight_offset(k, col, kk)


def test_blob_layout_is_a_bijection(orc):
    k, n = 96, 128
    offs = np.array([[orc.weight_offset(k, c, r) for r in range(k)] for c in range(n)])
    assert offs.min() == 128 and offs.max() == 128 + k * n - 1
    assert len(np.unique(offs)) == k * n


def test_pack_unpack_round_trip(orc):
    k, n = 160, 192
    w = orc.int8_uniform(n * k, -128, 127, 9).reshape(n, k)
    blob = orc.pack_blob(w, np.ones(n, np.float32))
    assert np.array_equal(orc.unpack_weights(blob, k, n), w)
    assert len(blob) == 128 + k * n + 8 * n + 4 * k


def test_header_checks(orc):
    """reference op_executor.cc:331-335: any field off -> -3."""
    k, n = 64, 128
    blob = orc.pack_blob(np.zeros((n, k), np.int8), np.ones(n, np.float32))
    assert orc.check_header(blob, k, n) == 0
    for field in range(9):
        bad = blob.copy()
        v = np.frombuffer(bad[:36].tobytes(), np.uint32).copy()
        v[field] += 1
        bad[:36] = np.frombuffer(v.tobytes(), np.uint8)
        assert orc.check_header(bad, k, n) == -3
    assert orc.check_header(blob, k + 32, n) == -3


# ---------------------------------------------------------- int32 arithmetic ----

def test_accumulate_brute_force(orc):
    rng = np.random.default_rng(3)
    for m, k, n in [(5, 64, 64), (7, 96, 128), (3, 1024, 64)]:
        w = rng.integers(-128, 128, (n, k)).astype(np.int8)
        u = rng.integers(0, 256, (m, k)).astype(np.uint8)
        blob = orc.pack_blob(w, np.ones(n, np.float32))
        acc = orc.accumulate(u, blob, k, n)
        ref = u.astype(np.int64) @ w.astype(np.int64).T
        assert np.array_equal(acc, ref.astype(np.int32))


def test_one_hot_layout(orc):
    """One-hot cases on the model of reference integer_tests.c:249-275."""
    k, n = 64, 64
    for (r, kk, col) in [(0, 0, 0), (3, 31, 17), (4, 32, 63), (1, 63, 32), (2, 5, 40)]:
        w = np.zeros((n, k), np.int8)
        w[col, kk] = 1
        u = np.zeros((5, k), np.uint8)
        u[r, kk] = 1
        acc = orc.accumulate(u, orc.pack_blob(w, np.ones(n, np.float32)), k, n)
        expect = np.zeros((5, n), np.int32)
        expect[r, col] = 1
        assert np.array_equal(acc, expect)


@pytest.mark.parametrize("target", [0, 1, -1, 32767, 32768, 32769, -32767, -32768, -32769, 65535, 65536, 65537,
                                    -65535, -65536, -65537, 131071, 131072, 1036320, -1036320])
def test_int32_boundary_targets(orc, target):
    """Boundary targets and construction of reference integer_tests.c:97-110."""
    k, n = 64, 64
    u = np.zeros((1, k), np.uint8)
    w = np.zeros((n, k), np.int8)
    rem, sign, i = abs(target), (-1 if target < 0 else 1), 0
    while rem >= 32385:
        u[0, i], w[0, i] = 255, sign * 127
        rem -= 32385
        i += 1
    if rem >= 127:
        u[0, i], w[0, i] = rem // 127, sign * 127
        rem %= 127
        i += 1
    if rem:
        u[0, i], w[0, i] = rem, sign
    acc = orc.accumulate(u, orc.pack_blob(w, np.ones(n, np.float32)), k, n)
    assert acc[0, 0] == target


def study_hash(x):
    x &= 0xffffffff
    x ^= x >> 16
    x = (x * 0x7feb352d) & 0xffffffff
    x ^= x >> 15
    x = (x * 0x846ca68b) & 0xffffffff
    return x ^ (x >> 16)


def study_a(r, k, seed):
    """Activation generator of reference tests/hmx-probe/study_data.h:4-12."""
    if seed == 0:
        return 129
    if seed in (30, 31):
        return 255
    return study_hash(r * 7919 + k * 13 + seed * 104729) & 255


def study_w(k, n, seed):
    """INT8 weight generator (kind 1) of reference tests/hmx-probe/study_data.h:13-20."""
    if seed == 0:
        return 1
    if seed == 30:
        return 127
    if seed == 31:
        return -128
    if 12 <= seed < 24:
        return (study_hash(k * 3571 + n * 23 + seed * 65537) & 255) - 128
    return (study_hash(k * 3571 + n * 23 + seed * 65537) & 15) - 8


@pytest.mark.parametrize("seed,kt", [(0, 1), (7, 4), (13, 4), (23, 1), (30, 48), (31, 48)])
def test_study_known_answers(orc, seed, kt):
    """reference study_host.c:66-72: raw = sum a*w and signed = sum (a-128)*w;
    the output path with sums = sum_k w, sw = 1, s = 1 must give exactly `signed`."""
    m, n, k = 64, 64, kt * 32
    a = np.array([[study_a(r, kk, seed) for kk in range(k)] for r in range(m)], np.int64)
    w = np.array([[study_w(kk, c, seed) for kk in range(k)] for c in range(n)], np.int64)
    raw = a @ w.T
    signed = (a - 128) @ w.T
    blob = orc.pack_blob(w.astype(np.int8), np.ones(n, np.float32))
    acc = orc.accumulate(a.astype(np.uint8), blob, k, n)
    assert np.array_equal(acc, raw.astype(np.int32))
    y = orc.output(acc, np.ones(m, np.float32), blob, k, n)
    assert np.array_equal(y, signed.astype(np.float32))


def test_zero_point_correction_padded(orc):
    """reference integer_tests.c:111-135: signed activation via zp=128,
    got - 128*colsum == sum (a-128)*w, on a padded 5 x 64 case."""
    m, n = 5, 64
    for kt in range(1, 5):
        k = kt * 32
        depth = k - 1
        a = np.full((m, k), 128, np.int64)
        w = np.zeros((n, k), np.int64)
        for r in range(m):
            for kk in range(depth):
                a[r, kk] = (r * 13 + kk * 17) % 256
        for kk in range(depth):
            for c in range(17):
                w[c, kk] = (kk * 11 + c * 5) % 16 - 8
        blob = orc.pack_blob(w.astype(np.int8), np.ones(n, np.float32))
        acc = orc.accumulate(a.astype(np.uint8), blob, k, n)
        got = acc.astype(np.int64) - 128 * w.sum(axis=1)[None, :]
        assert np.array_equal(got, (a - 128) @ w.T)


def test_output_wraps_and_scales(orc):
    """c = acc - (sums << 7) in int32 two's complement; y = (c*sw)*s."""
    m, k, n = 3, 64, 64
    rng = np.random.default_rng(5)
    acc = rng.integers(-2**31, 2**31, (m, n)).astype(np.int32)
    sums = rng.integers(-2**31, 2**31, n).astype(np.int32)
    sw = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    s = rng.uniform(1e-3, 1.0, m).astype(np.float32)
    blob = orc.pack_blob(np.zeros((n, k), np.int8), sw, sums=sums)
    y = orc.output(acc, s, blob, k, n)
    c = (acc.astype(np.int64) - (sums.astype(np.int64) << 7)) & 0xffffffff
    c = c.astype(np.uint32).view(np.int32)
    ref = (c.astype(np.float32) * sw[None, :]).astype(np.float32) * s[:, None]
    assert np.array_equal(y.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    # identity sw = 1, s = 1 gives (float)c
    blob1 = orc.pack_blob(np.zeros((n, k), np.int8), np.ones(n, np.float32), sums=np.zeros(n, np.int32))
    assert np.array_equal(orc.output(acc, np.ones(m, np.float32), blob1, k, n), acc.astype(np.float32))


def test_linear_composes_stages(orc):
    m, k, n = 9, 96, 128
    x = orc.normal(m * k, 0, 1, 4).reshape(m, k)
    w = orc.int8_uniform(n * k, -127, 127, 5).reshape(n, k)
    inv = orc.uniform(k, 0.5, 2.0, 6)
    blob = orc.pack_blob(w, orc.uniform(n, 1e-4, 1e-3, 7), inv=inv)
    u, s = orc.quantize(x, inv)
    y = orc.output(orc.accumulate(u, blob, k, n), s, blob, k, n)
    assert np.array_equal(orc.linear(x, blob, k, n).view(np.uint32), y.view(np.uint32))
    assert np.array_equal(orc.linear(x, blob, k, n, nthreads=1).view(np.uint32), y.view(np.uint32))


def test_planes_reassemble(orc):
    """Raw-plane export: gathering each 32-column half back per reference
    linear_w8a8.c:209-227 (flat stream over rows x 128 bytes, plane p = byte p)
    restores the accumulator."""
    rng = np.random.default_rng(6)
    for m in (64, 77, 130):
        n = 64
        acc = rng.integers(-2**31, 2**31, (m, n)).astype(np.int32)
        out = orc.planes(acc).reshape(m, n * 4)
        back = np.zeros((m, n), np.uint32)
        for tile in range(0, m, 64):
            rows = min(64, m - tile)
            for n0 in range(0, n, 32):
                stream = out[tile:tile + rows, n0 * 4:n0 * 4 + 128].reshape(-1)
                planes = stream.reshape(4, rows, 32).astype(np.uint32)
                back[tile:tile + rows, n0:n0 + 32] = (planes[0] | planes[1] << 8 | planes[2] << 16 |
                                                      planes[3] << 24)
        assert np.array_equal(back.view(np.int32), acc)


# ------------------------------------------------------------------- F16 -------

def permuted_index_from_writer(k_total, r, c):
    """reference src/host/test.c:547-558 writer."""
    tile_idx = (c // 32) * (k_total // 32) + r // 32
    return tile_idx * 1024 + ((r % 32) & ~1) * 32 + (c % 32) * 2 + (r % 32 & 1)


def test_f16_permuted_index_matches_writer(orc):
    for k, n in [(64, 64), (96, 128)]:
        for r in range(k):
            for c in range(0, n, 3):
                assert orc.f16_permuted_index(k, r, c) == permuted_index_from_writer(k, r, c)


def test_f16_all_ones_gives_k(orc):
    m, k, n = 4, 96, 64
    perm = orc.f16_permute(np.ones((k, n), np.float16).view(np.uint16))
    y = orc.f16_gemm_epilogue(np.ones((m, k), np.float32), perm, None, m, k, n, n, 0)
    assert (y == k).all()


def test_f16_one_hot(orc):
    m, k, n = 3, 64, 64
    x = orc.normal(m * k, 0, 1, 8).reshape(m, k)
    for kk, col in [(0, 0), (33, 5), (63, 63), (17, 40)]:
        w = np.zeros((k, n), np.float16)
        w[kk, col] = 1.0
        y = orc.f16_gemm_epilogue(x, orc.f16_permute(w.view(np.uint16)), None, m, k, n, n, 0)
        expect = np.zeros((m, n), np.float32)
        expect[:, col] = x[:, kk].astype(np.float16).astype(np.float32)
        assert np.array_equal(y, expect)


def test_f16_matches_float64_reference(orc):
    m, k, n = 9, 256, 96
    x = orc.normal(m * k, 0, 1, 9).reshape(m, k)
    w = orc.normal(k * n, 0, 0.02, 10).reshape(k, n).astype(np.float16)
    y = orc.f16_gemm_epilogue(x, orc.f16_permute(w.view(np.uint16)), None, m, k, n, n, 0)
    exact = x.astype(np.float16).astype(np.float64) @ w.astype(np.float64)
    ref = exact.astype(np.float16).astype(np.float32)
    ulp = np.abs(ref.astype(np.float16).view(np.int16).astype(np.int32) -
                 y.astype(np.float16).view(np.int16).astype(np.int32))
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99


def test_gelu_closed_form(orc):
    """x*sigmoid(2u) == 0.5*x*(1 + tanh(u)), u = sqrt(2/pi)*(x + 0.044715 x^3):
    pins 1.5957691216057308 = 2*sqrt(2/pi) and the sigmoid orientation."""
    z = np.linspace(-12, 12, 4001).astype(np.float32)
    got = np.array([orc.gelu_tanh(v) for v in z], np.float64)
    zd = z.astype(np.float64)
    u = np.sqrt(2 / np.pi) * (zd + 0.044715 * zd**3)
    # tanh form where 1 + tanh(u) keeps its precision in double; below that the
    # equivalent z / (1 + exp(-2u)) is evaluated instead.
    ref = np.where(zd >= -5, 0.5 * zd * (1 + np.tanh(u)), zd / (1 + np.exp(-2 * u)))
    # Float evaluation: the argument a = 2u takes four roundings (cubic, sum,
    # gain), each costing up to |a| * 2^-24 relative in exp; the reference
    # floors the exp2 argument at -126 (mat_mul.c:800), so far negative inputs
    # give about z * 2^-126 instead of underflowing.
    tol = (2e-6 + np.abs(2 * u) * 2.0**-21) * np.abs(ref) + np.abs(zd) * 2.0**-125
    assert np.all(np.abs(got - ref) <= tol)


def test_quick_gelu_closed_form(orc):
    z = np.linspace(-30, 30, 6001).astype(np.float32)
    got = np.array([orc.quick_gelu(v) for v in z], np.float64)
    zd = z.astype(np.float64)
    ref = zd / (1 + np.exp(-1.702 * zd))
    tol = (2e-6 + np.abs(1.702 * zd) * 2.0**-23) * np.abs(ref) + np.abs(zd) * 2.0**-125
    assert np.all(np.abs(got - ref) <= tol)


def test_f16_modes_relations(orc):
    m, k, n = 7, 64, 96
    x = orc.normal(m * k, 0, 1, 11).reshape(m, k)
    perm = orc.f16_permute(orc.normal(k * n, 0, 0.02, 12).reshape(k, n).astype(np.float16).view(np.uint16))
    bias = orc.normal(n, 0, 0.02, 13)
    v = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
    z = orc.f16_gemm_epilogue(x, perm, bias, m, k, n, n, 0)
    assert np.array_equal(z, (v + bias[None, :]).astype(np.float32))
    g = orc.f16_gemm_epilogue(x, perm, bias, m, k, n, n, 1)
    assert np.array_equal(g, np.array([[orc.gelu_tanh(t) for t in row] for row in z], np.float32))
    q = orc.f16_gemm_epilogue(x, perm, bias, m, k, n, n, 2)
    assert np.array_equal(q, np.array([[orc.quick_gelu(t) for t in row] for row in z], np.float32))
    ch = 64
    t = orc.f16_gemm_epilogue(x, perm, bias[:ch].copy(), m, k, n, ch, 3)
    assert np.array_equal(t, z[:, :ch].T)


def test_generators_deterministic(orc):
    a = orc.normal(1000, 0, 1, 42)
    assert np.array_equal(a, orc.normal(1000, 0, 1, 42))
    assert abs(a.mean()) < 0.1 and abs(a.std() - 1) < 0.1
    w = orc.int8_uniform(100000, -127, 127, 1)
    assert w.min() == -127 and w.max() == 127 and abs(w.astype(float).mean()) < 1.0
