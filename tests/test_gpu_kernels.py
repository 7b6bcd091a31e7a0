"""GPU parity of the hb_* kernels against the CPU oracle, called through the C ABI.

Bar: quantized activations, row scales, int32 accumulators and W8A8 f32
outputs bit-exact; the W8A8 GELU extension within 1e-5 relative (libm exp2f vs
device exp2f); F16 GEMM + epilogues within the bound of tests/tolerances.py
(2e-3 relative to the fp16-rounded magnitude, plus fp32 accumulation error
where the dot product cancels).
"""
import numpy as np
import pytest

from tolerances import assert_f16_close, f16_abs_dot

pytestmark = pytest.mark.gpu


def make_w8a8(orc, m, k, n, seed, inv_kind="ones", sums_kind="exact", scale_lo=1e-4, scale_hi=1e-3, outliers=0.0):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    if outliers:
        rng = np.random.default_rng(seed + 7)
        chans = rng.choice(k, max(1, int(outliers * k)), replace=False)
        x[:, chans] *= 20.0
    w = orc.int8_uniform(n * k, -127, 127, seed + 1).reshape(n, k)
    sw = orc.uniform(n, scale_lo, scale_hi, seed + 2)
    inv = None
    if inv_kind == "uniform":
        inv = orc.uniform(k, 0.5, 2.0, seed + 3)
    sums = None
    if sums_kind == "random":
        sums = np.random.default_rng(seed + 4).integers(-2**20, 2**20, n).astype(np.int32)
    blob = orc.pack_blob(w, sw, sums=sums, inv=inv, signature=seed)
    return x, w, blob


def upload_blob(hip, blob):
    return hip.DeviceBuffer.from_array(blob)


@pytest.mark.parametrize("m,k,inv_kind", [(77, 768, "ones"), (77, 768, "uniform"), (1, 96, "ones"), (5, 32, "uniform"),
                                          (33, 6144, "uniform"), (4, 14336, "ones"), (130, 1536, "uniform"),
                                          # one workgroup per row: up to 768 rows (1024 for rows past 2048
                                          # values) or rows past 6144 values
                                          (64, 1536, "uniform"), (65, 1536, "uniform"), (2, 2080, "uniform"),
                                          (3, 8192, "uniform"), (1, 16416, "ones"), (70, 14336, "uniform"),
                                          (2, 32768, "uniform"), (100, 480, "uniform"), (256, 4096, "ones"),
                                          (768, 1536, "uniform"), (1024, 4096, "uniform"), (2049, 8192, "uniform"),
                                          # 8-row blocks (769+ rows at up to 2048 values, 1025+ beyond),
                                          # ragged m and k % 64 == 32
                                          (1001, 480, "uniform"), (777, 1024, "ones"), (801, 1536, "uniform"),
                                          (1030, 2048, "uniform"), (1100, 3040, "uniform"), (1031, 4096, "uniform"),
                                          (1029, 6144, "uniform"), (1025, 5152, "uniform"),
                                          # from 2048 rows: 16-row blocks at one per CU (4096 x 1536 in the
                                          # baseline tests), else 8-row blocks with the smoothing vector in LDS
                                          (2100, 1536, "uniform"), (2048, 1248, "ones")])
def test_quantize_bit_exact(hip, orc, m, k, inv_kind):
    x, _, blob = make_w8a8(orc, m, k, 64, seed=m + k, inv_kind=inv_kind)
    x[0, :] = 0.0  # zero row: s = 1e-12, u = 128
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, 64)
    xd = hip.DeviceBuffer.from_array(x)
    inv_ptr = packed.ptr + hip.w8a8_packed_offset(k, 64, hip.SECTION_INV)
    q, s = hip.w8a8_quantize(xd, inv_ptr, m, k)
    kp = hip.kp_of(k)
    mp = (m + 15) // 16 * 16
    img = q.read(np.int8, mp * kp)
    rr, kk = np.meshgrid(np.arange(m), np.arange(kp), indexing="ij")
    tiled = ((rr // 16) * (kp // 64) + kk // 64) * 1024 + ((rr % 16) + 16 * ((kk % 64) // 16)) * 16 + kk % 16
    qh = img[tiled]
    sh = s.read(np.float32, m)
    inv = np.frombuffer(blob[128 + k * 64 + 8 * 64:].tobytes(), np.float32)[:k]
    u_ref, s_ref = orc.quantize(x, inv)
    np.testing.assert_array_equal(sh.view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal((qh[:, :k].astype(np.int16) + 128).astype(np.uint8), u_ref)
    assert not qh[:, k:].any()
    assert sh[0] == np.float32(1e-12) and (u_ref[0] == 128).all()


@pytest.mark.parametrize("k,n", [
    (96, 64),       # k % 64 == 32 exercises the zero padding; fewer 32-k blocks than waves
    (14336, 128),   # long k: every wave of a column group sums many blocks
    (4096, 1024),   # many column groups
])
def test_prepack_layout(hip, orc, k, n):
    _, w, blob = make_w8a8(orc, 2, k, n, seed=3, inv_kind="uniform", sums_kind="random")
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    kp = hip.kp_of(k)
    img = packed.read(np.int8, n * kp)
    nn, kk = np.meshgrid(np.arange(n), np.arange(kp), indexing="ij")
    idx = ((nn // 16) * (kp // 64) + kk // 64) * 1024 + ((nn % 16) + 16 * ((kk % 64) // 16)) * 16 + kk % 16
    expect = np.zeros((n, kp), np.int8)
    expect[:, :k] = w
    np.testing.assert_array_equal(img[idx], expect)
    sums = np.frombuffer(blob[128 + k * n + 4 * n:128 + k * n + 8 * n].tobytes(), np.int32)
    wsum = w.astype(np.int64).sum(axis=1)
    delta = packed.read(np.int32, n, hip.w8a8_packed_offset(k, n, hip.SECTION_DELTA))
    wsum128 = packed.read(np.int32, n, hip.w8a8_packed_offset(k, n, hip.SECTION_WSUM128))
    np.testing.assert_array_equal(delta, ((wsum - sums) * 128).astype(np.int64).astype(np.uint32).view(np.int32))
    np.testing.assert_array_equal(wsum128, (wsum * 128).astype(np.int32))
    sw = np.frombuffer(blob[128 + k * n:128 + k * n + 4 * n].tobytes(), np.float32)
    np.testing.assert_array_equal(packed.read(np.float32, n, hip.w8a8_packed_offset(k, n, hip.SECTION_SW)), sw)
    inv = np.zeros(kp, np.float32)
    inv[:k] = np.frombuffer(blob[128 + k * n + 8 * n:128 + k * n + 8 * n + 4 * k].tobytes(), np.float32)
    np.testing.assert_array_equal(packed.read(np.float32, kp, hip.w8a8_packed_offset(k, n, hip.SECTION_INV)), inv)


GEMM_SHAPES = [
    (5, 64, 128),      # small tile path, M tail
    (77, 768, 3072),   # C1
    (1, 4096, 1024),   # decode, 8-wave variant
    (4, 4096, 512),    # decode
    (16, 1024, 2048),  # decode, full 16 rows
    (16, 14336, 256),  # decode, K beyond the reference envelope
    (16, 4096, 14336),  # few rows, two column blocks per 16-wave workgroup (w8a8_decode_q)
    (3, 1504, 14336),  # w8a8_decode_q, three rows, K % 64 == 32
    (1, 96, 64),       # decode, K % 64 == 32
    (64, 14336, 4096),  # 17-128 rows, few output tiles: decode kernel per 16-row tile
    (72, 1056, 2048),  # the same, partial last row tile, K % 64 == 32
    (300, 1536, 768),  # tiled kernels (automatic shape choice from here on)
    (2048, 128, 2048),
    (4096, 64, 4096),
    (1000, 96, 4096),  # M tail and K % 64 == 32
    (4096, 1536, 6144),  # headline shape
]


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
def test_w8a8_raw_accumulator_bit_exact(hip, orc, m, k, n):
    x, _, blob = make_w8a8(orc, m, k, n, seed=m * 7 + n, inv_kind="uniform", sums_kind="random")
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    raw = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_gemm(raw, q, s, packed, m, k, n, hip.EPI_RAW)
    hip.sync()
    inv = np.frombuffer(blob[128 + k * n + 8 * n:].tobytes(), np.float32)[:k]
    u, _ = orc.quantize(x, inv)
    acc_ref = orc.accumulate(u, blob, k, n)
    np.testing.assert_array_equal(raw.read(np.int32, m * n).reshape(m, n), acc_ref)


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
def test_w8a8_linear_bit_exact(hip, orc, m, k, n):
    x, _, blob = make_w8a8(orc, m, k, n, seed=m + 3 * n + k, inv_kind="uniform", sums_kind="random",
                           outliers=0.01)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, xd, packed, m, k, n, ws)
    hip.sync()
    ref = orc.linear(x, blob, k, n)
    got = y.read(np.float32, m * n).reshape(m, n)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tile", range(6))
@pytest.mark.parametrize("m,k,n", [(261, 224, 960), (300, 1536, 576)])
def test_w8a8_every_tile_shape_bit_exact(hip, orc, tile, m, k, n):
    """Each tiled kernel instantiation, pinned in turn, with M, N and K tails
    (n = 960 is a multiple of 192 but not of 128 or 256)."""
    x, _, blob = make_w8a8(orc, m, k, n, seed=tile * 31 + m, inv_kind="uniform", sums_kind="random")
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    raw = hip.DeviceBuffer(m * n * 4)
    y = hip.DeviceBuffer(m * n * 4)
    prev = hip.w8a8_force_tile(tile)
    try:
        hip.w8a8_gemm(raw, q, s, packed, m, k, n, hip.EPI_RAW)
        hip.w8a8_gemm(y, q, s, packed, m, k, n, hip.EPI_SCALE)
        hip.sync()
    finally:
        hip.w8a8_force_tile(prev)
    inv = np.frombuffer(blob[128 + k * n + 8 * n:].tobytes(), np.float32)[:k]
    u, _ = orc.quantize(x, inv)
    np.testing.assert_array_equal(raw.read(np.int32, m * n).reshape(m, n), orc.accumulate(u, blob, k, n))
    ref = orc.linear(x, blob, k, n)
    got = y.read(np.float32, m * n).reshape(m, n)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


STREAM_TILE = 5  # hb_w8a8_force_tile index of the persistent streaming kernel
STREAM_WIDE_TILE = 6  # ... of its 256x192-tile form


@pytest.mark.parametrize("m,k,n", [
    (4096, 1536, 6144),  # headline: three 256x128 tiles per workgroup, one 16x16 block stored per k-step
    (1000, 320, 1088),   # fewest k-steps the kernel takes (5: four blocks stored per step); ragged M and N tiles
    (5000, 512, 4160),   # uneven tiles per workgroup (2 or 3), two blocks per step
    (777, 480, 2112),    # K % 64 == 32 (zero-padded k-step), 4 x 17 tiles: many workgroups without a tile
    (2304, 1088, 2112),  # 17 k-steps (one block per step, the last step stores none)
])
@pytest.mark.parametrize("epi", ["raw", "scale", "gelu"])
def test_w8a8_stream_kernel_bit_exact(hip, orc, m, k, n, epi):
    """The streaming kernel pinned: raw int32 accumulators and SCALE outputs
    bit-exact, GELU within 1e-5 relative of the oracle's GELU."""
    check_stream(hip, orc, STREAM_TILE, m, k, n, epi)


@pytest.mark.parametrize("m,k,n", [
    (4096, 1536, 6144),  # headline: two 256x192 tiles per workgroup
    (2048, 4096, 6144),  # C4 QKV: one tile per workgroup, 64 k-steps
    (1000, 256, 1152),   # fewest k-steps the 5-stage form takes (4); ragged M tiles
    (777, 480, 2304),    # K % 64 == 32 (zero-padded k-step), ragged M
    (5000, 1088, 4032),  # 17 k-steps, 20 x 21 tiles: 1 or 2 per workgroup
])
@pytest.mark.parametrize("epi", ["raw", "scale", "gelu"])
def test_w8a8_stream_wide_kernel_bit_exact(hip, orc, m, k, n, epi):
    """The 192-column streaming form pinned (GELU runs the 128-column form):
    the same bits as the oracle."""
    check_stream(hip, orc, STREAM_WIDE_TILE, m, k, n, epi)


def check_stream(hip, orc, tile, m, k, n, epi):
    x, _, blob = make_w8a8(orc, m, k, n, seed=m + k + n, inv_kind="uniform", sums_kind="random", outliers=0.01,
                           scale_lo=1e-3 if epi == "gelu" else 1e-4, scale_hi=1e-2 if epi == "gelu" else 1e-3)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    y = hip.DeviceBuffer(m * n * 4)
    y.fill(0xA5)
    epilogue = {"raw": hip.EPI_RAW, "scale": hip.EPI_SCALE, "gelu": hip.EPI_SCALE_GELU}[epi]
    prev = hip.w8a8_force_tile(tile)
    try:
        hip.w8a8_gemm(y, q, s, packed, m, k, n, epilogue)
        hip.sync()
    finally:
        hip.w8a8_force_tile(prev)
    inv = np.frombuffer(blob[128 + k * n + 8 * n:].tobytes(), np.float32)[:k]
    if epi == "raw":
        u, _ = orc.quantize(x, inv)
        np.testing.assert_array_equal(y.read(np.int32, m * n).reshape(m, n), orc.accumulate(u, blob, k, n))
        return
    ref = orc.linear(x, blob, k, n)
    got = y.read(np.float32, m * n).reshape(m, n)
    if epi == "scale":
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    else:
        np.testing.assert_allclose(got, orc.gelu_tanh_array(ref), rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("tile,n", [(STREAM_TILE, 1024), (STREAM_WIDE_TILE, 1152)])
def test_w8a8_stream_kernel_row_stride(hip, orc, tile, n):
    """Output rows with a stride past n (ldy > n): nothing outside the n
    columns of each row is written."""
    m, k, ldy = 600, 768, n + 16
    x, _, blob = make_w8a8(orc, m, k, n, seed=77, inv_kind="uniform", sums_kind="random")
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    y = hip.DeviceBuffer(m * ldy * 4)
    y.fill(0xA5)
    prev = hip.w8a8_force_tile(tile)
    try:
        hip.w8a8_gemm(y, q, s, packed, m, k, n, hip.EPI_SCALE, ldy=ldy)
        hip.sync()
    finally:
        hip.w8a8_force_tile(prev)
    got = y.read(np.uint32, m * ldy).reshape(m, ldy)
    np.testing.assert_array_equal(got[:, :n], orc.linear(x, blob, k, n).view(np.uint32))
    assert (got[:, n:] == 0xA5A5A5A5).all()


def test_w8a8_gemm_choice_names_the_kernel(hip):
    """hb_w8a8_gemm_choice reports the path hb_w8a8_gemm takes: the decode
    kernel up to 16 rows, the per-row-tile decode kernel for few output
    tiles, the streaming kernel at the headline (768 tiles, 3 per CU), a
    pinned tile shape, and HB_E_INVAL for a bad shape."""
    lib = hip.lib()
    assert lib.hb_w8a8_gemm_choice(1, 4096, 14336) == hip.W8A8_CHOICE_DECODE
    assert lib.hb_w8a8_gemm_choice(16, 14336, 4096) == hip.W8A8_CHOICE_DECODE
    assert lib.hb_w8a8_gemm_choice(32, 4096, 4096) == hip.W8A8_CHOICE_DECODE_TILES
    assert lib.hb_w8a8_gemm_choice(4096, 1536, 6144) == hip.W8A8_STREAM_WIDE_TILE
    assert hip.w8a8_gemm_kernel(4096, 1536, 6144) == "w8a8_gemm_stream<256,192>"
    # 192-column tiles only where they fill whole rounds of CUs
    assert hip.w8a8_gemm_kernel(4096, 6144, 1536) == "w8a8_gemm_stream<256,128>"
    prev = hip.w8a8_force_tile(0)
    try:
        assert lib.hb_w8a8_gemm_choice(4096, 1536, 6144) == 0
        assert hip.w8a8_gemm_kernel(4096, 1536, 6144) == "w8a8_gemm_tiles<128,192>"
    finally:
        hip.w8a8_force_tile(prev)
    assert lib.hb_w8a8_gemm_choice(0, 1536, 6144) == -22


# One row: hb_w8a8_linear quantizes inside the weight-streaming kernel
# (one variant per kp range: <= 4096, <= 8192, <= 16384; for kp <= 4096 and
# at least one block per CU, two column blocks per workgroup).
DECODE_FUSED_SHAPES = [
    (1, 32, 64),       # smallest K (k % 64 == 32)
    (1, 4096, 14336),  # BASELINE decode gate/up shape (two blocks per workgroup)
    (1, 4064, 14272),  # two blocks per workgroup, row shorter than the threads
    (1, 3104, 8192),   # two blocks per workgroup, 49 of 64 tiles per block present
    (1, 4096, 12288),  # one block per workgroup (three per CU)
    (1, 2048, 9216),   # 5 half blocks per workgroup (w8a8_decode_even)
    (1, 1568, 10240),  # 5 half blocks per workgroup, k % 64 == 32
    (1, 2016, 14272),  # 7 half blocks per workgroup (odd starts), a short last workgroup, row shorter than the threads
    (1, 14336, 4096),  # BASELINE decode down shape
    (1, 4160, 256),    # just past the first variant
    (1, 8192, 512),
    (1, 16384, 128),
    (1, 1568, 1024),   # k % 64 == 32 with clamped tail tiles
]


@pytest.mark.parametrize("m,k,n", DECODE_FUSED_SHAPES)
def test_w8a8_decode_fused_bit_exact(hip, orc, m, k, n):
    x, _, blob = make_w8a8(orc, m, k, n, seed=k + n, inv_kind="uniform", sums_kind="random", outliers=0.01,
                           scale_lo=5e-5, scale_hi=5e-4)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, xd, packed, m, k, n, ws)
    hip.sync()
    ref = orc.linear(x, blob, k, n)
    np.testing.assert_array_equal(y.read(np.uint32, m * n).reshape(m, n), ref.view(np.uint32))


@pytest.mark.parametrize("m,k,n,gelu,check_oracle", [
    (77, 8192, 1024, False, True),    # 128 k-steps: eight slices of 16
    (40, 8224, 512, True, False),     # 129 k-steps in slices of 17: a short last slice
    (200, 5120, 512, False, True),    # 80 k-steps over 129-256 rows: two row tiles
    (100, 8192, 1088, True, False),   # n % 128 == 64: a last tile half past n
])
def test_w8a8_linear_splitk_bit_exact(hip, orc, m, k, n, gelu, check_oracle):
    """33-256 rows with few output tiles: with hb_w8a8_linear_workspace_bytes
    the GEMM splits K over int32 slices, which add exactly, so the result
    equals the one-pass GEMM (the smaller workspace) bit for bit."""
    big, small = hip.w8a8_linear_workspace_bytes(m, k, n), hip.w8a8_workspace_bytes(m, k)
    assert big > small
    x, _, blob = make_w8a8(orc, m, k, n, seed=k + n + m, inv_kind="uniform", sums_kind="random", outliers=0.01)
    x[m - 1] *= 7.0
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    epi = hip.EPI_SCALE_GELU if gelu else hip.EPI_SCALE
    y1, y2 = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4)
    y1.fill(0xFF)
    hip.w8a8_linear(y1, xd, packed, m, k, n, hip.DeviceBuffer(big), epilogue=epi)
    hip.w8a8_linear(y2, xd, packed, m, k, n, hip.DeviceBuffer(small), epilogue=epi)
    hip.sync()
    got = y1.read(np.uint32, m * n)
    np.testing.assert_array_equal(got, y2.read(np.uint32, m * n))
    if check_oracle:
        np.testing.assert_array_equal(got.reshape(m, n), orc.linear(x, blob, k, n).view(np.uint32))


@pytest.mark.parametrize("m,k,n", [
    (2, 4096, 14336),   # two rows, C5 gate/up shape
    (4, 4096, 14336),   # four rows
    (3, 1568, 1024),    # three rows (one zero A row), k % 64 == 32
    (4, 32, 64),        # smallest K
    (4, 4064, 14272),   # row shorter than the threads
])
def test_w8a8_decode_rows_bit_exact(hip, orc, m, k, n):
    """Two to four rows: quantization fused into the weight stream as well."""
    x, _, blob = make_w8a8(orc, m, k, n, seed=k + n + m, inv_kind="uniform", sums_kind="random", outliers=0.01,
                           scale_lo=5e-5, scale_hi=5e-4)
    x[m - 1] *= 7.0  # rows with different scales
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, hip.DeviceBuffer.from_array(x), packed, m, k, n, ws)
    hip.sync()
    ref = orc.linear(x, blob, k, n)
    np.testing.assert_array_equal(y.read(np.uint32, m * n).reshape(m, n), ref.view(np.uint32))


@pytest.mark.parametrize("m,k,n,gelu", [
    (77, 768, 3072, False),   # BASELINE C1: 64-column workgroups
    (5, 1536, 2048, True),    # fewest rows, longest k of the path, GELU
    (128, 1504, 192, False),  # k % 64 == 32, few column groups: 16-column workgroups
    (77, 32, 64, True),       # smallest K
    (100, 768, 2048, False),  # rows past m in the last 16-row tile
])
def test_w8a8_small_bit_exact(hip, orc, m, k, n, gelu):
    """5 <= m <= 128, k <= 1536: one launch that quantizes its own rows."""
    x, _, blob = make_w8a8(orc, m, k, n, seed=m + k + n, inv_kind="uniform", sums_kind="random", outliers=0.01,
                           scale_lo=1e-3 if gelu else 1e-4, scale_hi=1e-2 if gelu else 1e-3)
    x[::7] *= 5.0  # rows with different scales
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, hip.DeviceBuffer.from_array(x), packed, m, k, n, ws,
                    epilogue=hip.EPI_SCALE_GELU if gelu else hip.EPI_SCALE)
    hip.sync()
    ref = orc.linear(x, blob, k, n)
    if gelu:
        ref = orc.gelu_tanh_array(ref)
        got = y.read(np.float32, m * n).reshape(m, n)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30)
    else:
        np.testing.assert_array_equal(y.read(np.uint32, m * n).reshape(m, n), ref.view(np.uint32))


def test_w8a8_decode_fused_special_rows(hip, orc):
    """Zero row (s = 1e-12, u = 128), a row whose absmax is exactly 127
    (s = 1, so u = rint(t + 128)), and halves that round to even."""
    k, n = 256, 128
    _, _, blob = make_w8a8(orc, 1, k, n, seed=17, sums_kind="random")
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(1, k))
    rows = [np.zeros(k, np.float32),
            np.linspace(-127.0, 127.0, k, dtype=np.float32),
            np.where(np.arange(k) % 3 == 0, 0.5, np.where(np.arange(k) % 3 == 1, 1.5, 2.5)).astype(np.float32)]
    rows[2][0] = 127.0
    for row in rows:
        x = row.reshape(1, k)
        y = hip.DeviceBuffer(n * 4)
        hip.w8a8_linear(y, hip.DeviceBuffer.from_array(x), packed, 1, k, n, ws)
        hip.sync()
        np.testing.assert_array_equal(y.read(np.uint32, n), orc.linear(x, blob, k, n).view(np.uint32).ravel())


@pytest.mark.parametrize("m,k,n", [(77, 768, 3072), (4, 1536, 1024), (1000, 96, 4096), (1, 4096, 2048)])
def test_w8a8_gelu_epilogue(hip, orc, m, k, n):
    x, _, blob = make_w8a8(orc, m, k, n, seed=11, scale_lo=1e-3, scale_hi=1e-2)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_linear(y, xd, packed, m, k, n, ws, epilogue=hip.EPI_SCALE_GELU)
    hip.sync()
    ref = orc.gelu_tanh_array(orc.linear(x, blob, k, n))
    got = y.read(np.float32, m * n).reshape(m, n)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30)


@pytest.mark.parametrize("m,k,n,epi", [(300, 1536, 576, "scale"), (77, 768, 3072, "gelu"), (1, 4096, 1024, "scale")])
def test_w8a8_readout_equals_fused_epilogue(hip, orc, m, k, n, epi):
    """hb_w8a8_readout over the EPI_RAW sums gives the fused epilogue's bits
    (the profile-mode-2 split of MAC from readout)."""
    x, _, blob = make_w8a8(orc, m, k, n, seed=m + 3, inv_kind="uniform", sums_kind="random",
                           scale_lo=1e-3 if epi == "gelu" else 1e-4, scale_hi=1e-2 if epi == "gelu" else 1e-3)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    epilogue = hip.EPI_SCALE if epi == "scale" else hip.EPI_SCALE_GELU
    raw, fused, split = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4)
    hip.w8a8_gemm(raw, q, s, packed, m, k, n, hip.EPI_RAW)
    hip.w8a8_gemm(fused, q, s, packed, m, k, n, epilogue)
    hip.w8a8_readout(split, raw, s, packed, m, k, n, epilogue)
    hip.sync()
    got = split.read(np.uint32, m * n)
    np.testing.assert_array_equal(got, fused.read(np.uint32, m * n))
    if epi == "scale":
        np.testing.assert_array_equal(got.reshape(m, n), orc.linear(x, blob, k, n).view(np.uint32))


def test_w8a8_planes_export(hip, orc):
    m, k, n = 77, 64, 128
    x, _, blob = make_w8a8(orc, m, k, n, seed=5)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    q, s = hip.w8a8_quantize(xd, packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV), m, k)
    raw = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_gemm(raw, q, s, packed, m, k, n, hip.EPI_RAW)
    planes = hip.DeviceBuffer(m * n * 4)
    hip.w8a8_planes_from_raw(planes, raw, m, n)
    hip.sync()
    acc = raw.read(np.int32, m * n).reshape(m, n)
    np.testing.assert_array_equal(planes.read(np.uint8, m * n * 4), orc.planes(acc))


def f16_case(orc, m, k, n, seed, bias=True):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    w = orc.normal(k * n, 0.0, 0.02, seed + 1).reshape(k, n).astype(np.float16)
    perm = orc.f16_permute(w.view(np.uint16))
    b = orc.normal(n, 0.0, 0.02, seed + 2) if bias else None
    return x, w, perm, b


@pytest.mark.parametrize("m,k,n,mode,channels,bias", [
    (77, 768, 3072, 2, 3072, True),   # C2 first GEMM: QuickGELU
    (77, 3072, 768, 0, 768, True),    # C2 second GEMM: bias only
    (77, 768, 3072, 1, 3072, True),   # GELU
    (77, 768, 3072, 1, 3072, False),  # GELU without bias
    (64, 96, 64, 0, 64, False),       # opcode-1 semantics, K % 64 == 32
    (300, 256, 512, 3, 480, True),    # channel-major store, channels < n
    (1024, 256, 4096, 0, 4096, True), # 128x128 tiles
    (1, 128, 32, 2, 32, True),
    (128, 3072, 768, 3, 704, True),   # eight row fragments, channel-major, split-K
    (17, 1024, 96, 1, 96, False),     # two row fragments, a single split
    (48, 4096, 2048, 2, 2048, True),  # three row fragments -> four-fragment variant
    (64, 4096, 4096, 0, 4096, True),  # as many 32x32 tiles as CUs: split-K with a workspace
    (77, 1280, 5120, 1, 5120, True),  # 13 MB of weights: the split-K ring path rather than one launch
    (100, 10240, 512, 3, 480, True),  # long K, channel-major, split-K ring path
    (200, 4096, 1024, 2, 1024, True), # two 128-row tiles on the split-K ring path
    (1030, 512, 384, 3, 300, True),   # ring kernel, channel-major, m % 4 != 0: element stores
    (600, 2048, 256, 3, 200, True),   # split-K ring from 257 rows: channel-major slices, channels < n
    (999, 4096, 512, 3, 512, True),   # the same with m % 4 != 0 (element stores in the readout)
    (1000, 2304, 384, 1, 384, True),  # split-K ring from 257 rows, row-major, GELU
    (256, 11520, 1280, 3, 1280, True),  # a 512x512 UNet's 16x16 3x3 convolution at full size (im2col)
])
@pytest.mark.parametrize("split_k", [False, True])
def test_f16_gemm_epilogue(hip, orc, m, k, n, mode, channels, bias, split_k):
    """Tiled path, and (split_k) hb_f16_gemm_ws with its workspace: the
    split-K paths, the ring kernel or the tiled path as the shape selects."""
    ws_bytes = hip.f16_workspace_bytes(m, k, n)
    if split_k and not ws_bytes:
        pytest.skip("m > 128: hb_f16_gemm_ws takes the tiled path")
    x, w, perm, b = f16_case(orc, m, k, n, seed=m + n + mode, bias=bias)
    permd = hip.DeviceBuffer.from_array(perm)
    packed = hip.f16_prepack(permd, k, n)
    xd = hip.DeviceBuffer.from_array(x)
    bd = hip.DeviceBuffer.from_array(b[:channels] if b is not None else np.zeros(1, np.float32)) if bias else None
    out_elems = m * (channels if mode == 3 else n)
    y = hip.DeviceBuffer(out_elems * 4)
    ws = hip.DeviceBuffer(ws_bytes) if split_k else None
    hip.f16_gemm(y, xd, packed, bd, m, k, n, channels, mode, workspace=ws)
    hip.sync()
    got = y.read(np.float32, out_elems)
    ref = orc.f16_gemm_epilogue(x, perm, None if b is None else b[:channels].copy() if mode == 3 else b, m, k, n,
                                channels, mode)
    v_ref = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
    absdot = f16_abs_dot(x, w)
    if mode == 3:
        got = got.reshape(channels, m)
        v_ref = v_ref.T[:channels]
        absdot = absdot.T[:channels]
        bias_cols = np.abs(b[:channels])[:, None] if b is not None else 0.0
    else:
        got = got.reshape(m, n)
        bias_cols = np.abs(b)[None, :] if b is not None else 0.0
    rel = assert_f16_close(got, ref, v_ref, bias_cols, absdot, k)
    # the north star's figure: the largest relative error where nothing cancels
    print(f"f16 {m}x{k}x{n} mode {mode} split_k {split_k}: max relative error {rel:.3g}")
    assert rel <= 2e-3


@pytest.mark.parametrize("m,k,n,mode,bias,check_oracle", [
    (512, 4096, 1024, 0, True, True),     # 128x128 tiles
    (1024, 1536, 3072, 2, True, False),   # 128x192 tiles, QuickGELU
    (300, 4096, 2048, 1, False, True),    # rows past m in the last tile, GELU
    (640, 2048, 1600, 0, True, False),    # n % 128 != 0: columns past n in the last tile
    (100, 4096, 14336, 2, True, False),   # few rows, 64x64 tiles
])
def test_f16_ring_matches_tiles(hip, orc, m, k, n, mode, bias, check_oracle):
    """Large M with a workspace: the fp16 activation image and the
    direct-to-LDS ring give the same bits as the tiled kernel (same MFMA
    sequence per accumulator), and stay within the F16 bound of the oracle."""
    ws_bytes = hip.f16_workspace_bytes(m, k, n)
    assert ws_bytes >= ((m + 15) // 16 * 16) * k * 2
    x, w, perm, b = f16_case(orc, m, k, n, seed=m + k + n, bias=bias)
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    bd = hip.DeviceBuffer.from_array(b) if bias else None
    y_ring, y_tiles = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4)
    prev, prev_split = hip.f16_force_stream(0), hip.f16_force_splitk(0)
    try:
        hip.f16_gemm(y_ring, xd, packed, bd, m, k, n, n, mode, workspace=hip.DeviceBuffer(ws_bytes))
    finally:
        hip.f16_force_stream(prev)
        hip.f16_force_splitk(prev_split)
    hip.f16_gemm(y_tiles, xd, packed, bd, m, k, n, n, mode)
    hip.sync()
    got = y_ring.read(np.uint32, m * n)
    np.testing.assert_array_equal(got, y_tiles.read(np.uint32, m * n))
    if check_oracle:
        ref = orc.f16_gemm_epilogue(x, perm, b, m, k, n, n, mode)
        v_ref = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
        bias_cols = np.abs(b)[None, :] if b is not None else 0.0
        assert_f16_close(got.view(np.float32).reshape(m, n), ref, v_ref, bias_cols, f16_abs_dot(x, w), k)


@pytest.mark.parametrize("m,k,n,mode,bias,check_oracle", [
    (512, 256, 1024, 0, True, True),      # one tile per workgroup
    (700, 160, 576, 1, False, True),      # rows past m, columns past n, k at the 6-stage minimum, GELU
    (700, 192, 640, 2, True, True),       # QuickGELU
    (4096, 256, 3072, 0, False, False),   # 384 tiles: some workgroups take two
    (4096, 320, 4096, 2, True, False),    # two whole rounds: the odd slots start late
    (4096, 256, 6144, 1, True, False),    # three rounds, GELU
    (2048, 1536, 1152, 0, True, False),   # long k, few tiles
    (333, 224, 2080, 2, True, True),      # n % 128 == 32: a last tile of one column pair, its bias clamped
    (256, 256, 8192, 1, True, False),     # one 256-row tile: 256 x 64 streaming tiles
])
def test_f16_stream_matches_ring(hip, orc, m, k, n, mode, bias, check_oracle):
    """The persistent streaming F16 kernel gives the same bits as the ring
    kernel (same MFMA sequence per output element, weights as the first
    operand) and stays within the F16 bound of the oracle."""
    ws = hip.DeviceBuffer(hip.f16_workspace_bytes(m, k, n))
    x, w, perm, b = f16_case(orc, m, k, n, seed=m + k + n + 7, bias=bias)
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    bd = hip.DeviceBuffer.from_array(b) if bias else None
    y_stream, y_ring = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * n * 4)
    y_stream.fill(0xFF)
    prev = hip.f16_force_stream(1)
    try:
        hip.f16_gemm(y_stream, xd, packed, bd, m, k, n, n, mode, workspace=ws)
        hip.f16_force_stream(0)
        hip.f16_gemm(y_ring, xd, packed, bd, m, k, n, n, mode, workspace=ws)
    finally:
        hip.f16_force_stream(prev)
    hip.sync()
    got = y_stream.read(np.uint32, m * n)
    np.testing.assert_array_equal(got, y_ring.read(np.uint32, m * n))
    if check_oracle:
        ref = orc.f16_gemm_epilogue(x, perm, b, m, k, n, n, mode)
        v_ref = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
        bias_cols = np.abs(b)[None, :] if b is not None else 0.0
        assert_f16_close(got.view(np.float32).reshape(m, n), ref, v_ref, bias_cols, f16_abs_dot(x, w), k)


@pytest.mark.parametrize("m,k,n,channels,mode,bias,check_oracle", [
    (4096, 1152, 128, 128, 3, True, True),      # VAE-like: channel-major, one 128-column chunk, 36 k-steps
    (1000, 96, 256, 200, 3, True, True),        # channels < n, three k-steps
    (997, 352, 128, 128, 3, False, True),       # m % 4 != 0: element stores; 11 k-steps (a tail of two)
    (2050, 320, 96, 96, 0, True, True),         # row-major, n under one chunk, 10 k-steps (a tail of one)
    (1500, 288, 320, 320, 1, True, True),       # two column chunks (256 + 64), GELU
    (4096, 2304, 256, 256, 2, False, False),    # QuickGELU, 72 k-steps
    (64, 32, 64, 64, 0, True, True),            # one k-step: fewer than the prefetch depth
    (3000, 1152, 512, 384, 3, True, False),     # two chunks, channel-major, channels < n
    # 128-row workgroups of 8 waves (row blocks x chunks fill the CUs)
    (32818, 96, 128, 128, 3, True, True),       # ragged m (m % 128 == 50), one chunk
    (16384, 64, 512, 448, 3, True, False),      # two chunks of one row block on one XCD (bid, bid + 8)
    (16400, 160, 256, 256, 1, True, False),     # row-major, 129 row blocks, GELU
])
def test_f16_xstream_matches_other_paths(hip, orc, m, k, n, channels, mode, bias, check_oracle):
    """The activation-streaming F16 kernel (fp32 rows read once, converted in
    registers) gives the same bits as the automatic choice without it (the
    same v_mfma_f32_16x16x32_f16 sequence per output element) and stays
    within the F16 bound of the oracle, in both output layouts."""
    ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, n), 256))
    x, w, perm, b = f16_case(orc, m, k, n, seed=m + k + n + 11, bias=bias)
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    bvec = None if b is None else (b[:channels].copy() if mode == 3 else b)
    bd = hip.DeviceBuffer.from_array(bvec) if bias else None
    out_elems = m * (channels if mode == 3 else n)
    y_x, y_o = hip.DeviceBuffer(out_elems * 4), hip.DeviceBuffer(out_elems * 4)
    y_x.fill(0xFF)
    prev = hip.f16_force_xstream(1)
    try:
        hip.f16_gemm(y_x, xd, packed, bd, m, k, n, channels, mode, workspace=ws)
        hip.f16_force_xstream(0)
        hip.f16_gemm(y_o, xd, packed, bd, m, k, n, channels, mode, workspace=ws)
    finally:
        hip.f16_force_xstream(prev)
    hip.sync()
    got = y_x.read(np.uint32, out_elems)
    np.testing.assert_array_equal(got, y_o.read(np.uint32, out_elems))
    if check_oracle:
        ref = orc.f16_gemm_epilogue(x, perm, bvec, m, k, n, channels, mode)
        v_ref = orc.f16_gemm_epilogue(x, perm, None, m, k, n, n, 0)
        absdot = f16_abs_dot(x, w)
        if mode == 3:
            gotf = got.view(np.float32).reshape(channels, m)
            v_ref, absdot = v_ref.T[:channels], absdot.T[:channels]
            bias_cols = np.abs(bvec)[:, None] if bias else 0.0
        else:
            gotf = got.view(np.float32).reshape(m, n)
            bias_cols = np.abs(b)[None, :] if bias else 0.0
        assert_f16_close(gotf, ref, v_ref, bias_cols, absdot, k)


@pytest.mark.parametrize("m,k,n,channels,ring", [
    (1030, 512, 384, 300, True),    # ring kernel (k < 2048), m % 4 != 0
    (2500, 1024, 1024, 1000, True), # ring kernel, 160 tiles of 128 x 128
    (600, 2048, 256, 200, False),   # split-K ring from 257 rows
    (999, 4096, 512, 512, False),   # split-K ring, m % 4 != 0
    (2048, 5760, 640, 640, False),  # split-K ring at kRingSplitRows, 80 tiles
])
def test_f16_channel_major_matches_row_major(hip, orc, m, k, n, channels, ring):
    """Mode 3 (channel-major y[channels][m]) gives the bits of mode 0's output
    transposed on the same path, and on the ring kernel also the bits of the
    tiled kernel (hb_f16_gemm without a workspace)."""
    ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, n), 256))
    x, w, perm, b = f16_case(orc, m, k, n, seed=m + k + n + 5, bias=True)
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, n)
    xd = hip.DeviceBuffer.from_array(x)
    bd_rows, bd_ch = hip.DeviceBuffer.from_array(b), hip.DeviceBuffer.from_array(b[:channels].copy())
    y0, y3, yt = hip.DeviceBuffer(m * n * 4), hip.DeviceBuffer(m * channels * 4), hip.DeviceBuffer(m * channels * 4)
    y3.fill(0xFF)
    hip.f16_gemm(y0, xd, packed, bd_rows, m, k, n, n, 0, workspace=ws)
    hip.f16_gemm(y3, xd, packed, bd_ch, m, k, n, channels, 3, workspace=ws)
    if ring:
        hip.f16_gemm(yt, xd, packed, bd_ch, m, k, n, channels, 3)
    hip.sync()
    rows = y0.read(np.uint32, m * n).reshape(m, n)
    got = y3.read(np.uint32, m * channels).reshape(channels, m)
    np.testing.assert_array_equal(got, np.ascontiguousarray(rows.T[:channels]))
    if ring:
        np.testing.assert_array_equal(got, yt.read(np.uint32, m * channels).reshape(channels, m))


def test_f16_workspace_covers_only_the_paths_that_run(hip):
    """The workspace holds split-K slices only for shapes that take the
    split-K ring path: many output tiles at 2048 rows need the fp16 image
    alone, few tiles at k >= 2048 the image and the slices."""
    image = lambda m, k: ((m + 15) // 16 * 16 * k * 2 + 255) // 256 * 256
    assert hip.f16_workspace_bytes(2048, 1024, 14336) == image(2048, 1024)
    assert hip.f16_workspace_bytes(2048, 2048, 14336) == image(2048, 2048)
    assert hip.f16_workspace_bytes(1024, 4608, 512) > image(1024, 4608) + 1024 * 512 * 4
    assert hip.f16_workspace_bytes(3000, 4608, 512) == image(3000, 4608)


def test_f16_all_ones_gives_k(hip, orc):
    m, k, n = 32, 256, 64
    x = np.ones((m, k), np.float32)
    perm = orc.f16_permute(np.ones((k, n), np.float16).view(np.uint16))
    packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, n)
    y = hip.DeviceBuffer(m * n * 4)
    hip.f16_gemm(y, hip.DeviceBuffer.from_array(x), packed, None, m, k, n, n, 0)
    hip.sync()
    assert (y.read(np.float32, m * n) == k).all()


@pytest.mark.parametrize("m,k,n", [(300, 256, 576), (1, 4096, 1024)])
def test_graph_replays_match_eager(hip, orc, m, k, n):
    """hb_w8a8_linear captured into a graph: every replay, with other eager
    work on the same workspace between replays, equals the eager result."""
    x, _, blob = make_w8a8(orc, m, k, n, seed=5, inv_kind="uniform", sums_kind="random")
    x2 = orc.normal(m * k, 0.0, 3.0, 6).reshape(m, k)
    packed = hip.w8a8_prepack(upload_blob(hip, blob), k, n)
    xd, x2d = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(x2)
    ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
    y_eager, y_graph, y_other = (hip.DeviceBuffer(m * n * 4) for _ in range(3))
    stream = hip.default_stream()
    hip.w8a8_linear(y_eager, xd, packed, m, k, n, ws, stream=stream)
    hip.sync()
    eager = y_eager.read(np.uint32, m * n)
    np.testing.assert_array_equal(eager.view(np.float32).reshape(m, n).view(np.uint32),
                                  orc.linear(x, blob, k, n).view(np.uint32))
    with hip.Graph.capture(stream) as graph:
        hip.w8a8_linear(y_graph, xd, packed, m, k, n, ws, stream=stream)
    for _ in range(4):
        y_graph.zero()
        hip.w8a8_linear(y_other, x2d, packed, m, k, n, ws, stream=stream)  # overwrites the workspace
        hip.sync()
        graph.launch(stream)
        hip.sync()
        np.testing.assert_array_equal(y_graph.read(np.uint32, m * n), eager)
