"""Opcode 19 (model auxiliary f32 ops): oracle pins, executor validation, GPU parity.

Reference semantics: src/dsp/ops/mat_mul.c:2356-2501 (kernels and task split),
src/dsp/op_executor.cc:371-404 (validation and buffer sizes).

- CPU: the oracle's restatement is pinned against independent numpy/float64
  closed forms (layer/RMS/group norm statistics, affine and modulation,
  broadcasts, transposes, 2x2 rotary matrices, gated products) and against
  invariants (normalized rows have mean 0 and variance 1, identity rotary
  matrices only change the layout, rotations keep pair norms); the executor's
  codes for every validation rule run without a GPU.
- GPU: hb_model_aux and opcode 19 against the oracle on the same inputs.
  Bit-exact where both sides do the same IEEE operations (broadcasts,
  transpose, modulation gate, rotary); the norms within 2 ulp-scale
  tolerance (double row sums in a different order); activations within 4e-6
  relative (GPU exp2f against libm exp2f).
"""
import numpy as np
import pytest

import htp_ops as h

ACT_RTOL, ACT_ATOL = 4e-6, 1e-6
NORM_RTOL, NORM_ATOL = 2e-6, 2e-6


def rng_normal(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def f64_sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def f64_act(v, act):
    v = v.astype(np.float64)
    if act == 1:
        return v * f64_sigmoid(1.5957691216057308 * (v + 0.044715 * v ** 3))
    if act == 2:
        return v * f64_sigmoid(1.702 * v)
    return v * f64_sigmoid(v)


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------

def test_oracle_layer_norm_closed_form(orc):
    rows, width = 5, 96
    x = rng_normal((rows, width), 1, 3.0) + 2.0
    w, b = rng_normal(width, 2), rng_normal(width, 3)
    y = orc.model_aux(x, w, b, 0, rows * width, width, other_count=width, eps=1e-6).reshape(rows, width)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    ref = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-6) * w + b
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=2e-6)
    # without affine: mean 0, variance 1
    z = orc.model_aux(x, None, None, 0, rows * width, width).reshape(rows, width).astype(np.float64)
    np.testing.assert_allclose(z.mean(1), 0.0, atol=1e-6)
    np.testing.assert_allclose(z.var(1), 1.0, rtol=1e-5)


def test_oracle_rms_norm_and_partial_rows(orc):
    width = 64
    x = rng_normal(3 * width + 10, 4, 2.0)
    w = rng_normal(width, 5)
    keep = np.full(x.size, 7.0, np.float32)
    y = orc.model_aux(x, w, None, 1, x.size, width, other_count=width, eps=0.0, out=keep)
    x3 = x[:3 * width].reshape(3, width).astype(np.float64)
    ref = x3 / np.sqrt((x3 ** 2).mean(1, keepdims=True)) * w
    np.testing.assert_allclose(y[:3 * width].reshape(3, width), ref, rtol=2e-6, atol=2e-6)
    # the tail past the last whole row is not written
    assert (y[3 * width:] == 7.0).all()


def test_oracle_group_norm(orc):
    batch, channels, groups, spatial = 2, 8, 4, 20
    x = rng_normal((batch, channels, spatial), 6, 1.5) - 0.5
    w, b = rng_normal(channels, 7), rng_normal(channels, 8)
    y = orc.model_aux(x, w, b, 2, x.size, spatial, channels=channels, spatial=spatial, groups=groups, batch=batch,
                      other_count=channels, eps=1e-5).reshape(batch, channels, spatial)
    g = x.astype(np.float64).reshape(batch, groups, -1)
    mu, var = g.mean(2, keepdims=True), g.var(2, keepdims=True)
    ref = ((g - mu) / np.sqrt(var + 1e-5)).reshape(batch, channels, spatial) * w[:, None] + b[:, None]
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("per_batch", [False, True])
def test_oracle_layer_norm_modulation(orc, per_batch):
    batch, tokens, width = 2, 3, 32
    x = rng_normal((batch, tokens, width), 9)
    other = width * batch if per_batch else width
    scale, shift = rng_normal(other, 10, 0.1), rng_normal(other, 11, 0.1)
    y = orc.model_aux(x, scale, shift, 9, x.size, width, spatial=tokens, batch=batch, other_count=other,
                      eps=1e-6).reshape(batch, tokens, width)
    x64 = x.astype(np.float64)
    mu = x64.mean(2, keepdims=True)
    n = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(2, keepdims=True) + 1e-6)
    s = scale.reshape(-1, 1, width) if per_batch else scale.reshape(1, 1, width)
    t = shift.reshape(-1, 1, width) if per_batch else shift.reshape(1, 1, width)
    np.testing.assert_allclose(y, n * (1.0 + s) + t, rtol=3e-6, atol=3e-6)


def test_oracle_norm_silu(orc):
    width = 48
    x = rng_normal(2 * width, 12)
    plain = orc.model_aux(x, None, None, 0, x.size, width)
    act = orc.model_aux(x, None, None, 0, x.size, width, activation=1)
    np.testing.assert_allclose(act, f64_act(plain, 4), rtol=ACT_RTOL, atol=ACT_ATOL)


def test_oracle_broadcasts_and_activations(orc):
    x = rng_normal(3 * 40, 13, 4.0)
    w = rng_normal(40, 14)
    assert np.array_equal(orc.model_aux(x, w, None, 3, x.size, 40, other_count=40), x + np.tile(w, 3))
    assert np.array_equal(orc.model_aux(x, w, None, 4, x.size, 40, other_count=40), x * np.tile(w, 3))
    for mode, act in ((5, 4), (6, 1), (7, 2)):
        np.testing.assert_allclose(orc.model_aux(x, None, None, mode, x.size, 40), f64_act(x, act), rtol=ACT_RTOL,
                                   atol=ACT_ATOL)
    # SiLU special values: 0 at 0, vanishing for large negative inputs, identity for large positive ones
    assert orc.silu(0.0) == 0.0 and abs(orc.silu(-200.0)) < 1e-30 and orc.silu(100.0) == 100.0


def test_oracle_transpose(orc):
    batch, width, spatial = 3, 5, 7
    x = rng_normal((batch, width, spatial), 15)
    y = orc.model_aux(x, None, None, 8, x.size, width, spatial=spatial, batch=batch)
    assert np.array_equal(y.reshape(batch, spatial, width), x.transpose(0, 2, 1))


@pytest.mark.parametrize("per_batch", [False, True])
def test_oracle_modulation_gate(orc, per_batch):
    batch, tokens, width = 2, 3, 16
    x = rng_normal((batch, tokens, width), 16)
    other = width * batch if per_batch else width
    w, b = rng_normal(other, 17), rng_normal(x.size, 18)
    y = orc.model_aux(x, w, b, 10, x.size, width, spatial=tokens, batch=batch, other_count=other)
    wb = w.reshape(-1, 1, width) if per_batch else w.reshape(1, 1, width)
    assert np.array_equal(y.reshape(batch, tokens, width), x * wb + b.reshape(batch, tokens, width))


def rope_matrices(batch_or_1, tokens, dim, seed, identity=False):
    ang = np.random.default_rng(seed).uniform(-np.pi, np.pi, (batch_or_1, tokens, dim // 2)).astype(np.float32)
    c, s = np.cos(ang), np.sin(ang)
    if identity:
        c, s = np.ones_like(c), np.zeros_like(s)
    return np.stack([c, -s, s, c], -1).astype(np.float32).ravel()  # [[c, -s], [s, c]] per pair


@pytest.mark.parametrize("groups", [1, 2])
def test_oracle_rope(orc, groups):
    batch, tokens, heads, dim = 2, 5, 3, 8
    x = rng_normal((batch, tokens, heads, dim), 19)
    pe = rope_matrices(groups, tokens, dim, 20)
    y = orc.model_aux(x, pe, None, 11, x.size, dim, channels=heads, spatial=tokens, groups=groups, batch=batch,
                      other_count=2 * dim * tokens * groups).reshape(batch, heads, tokens, dim)
    m = pe.reshape(groups, tokens, dim // 2, 4)
    mb = np.broadcast_to(m, (batch, tokens, dim // 2, 4)) if groups == 1 else m
    x0, x1 = x[..., 0::2], x[..., 1::2]  # [batch][token][head][pair]
    m4 = mb[:, :, None, :, :]
    r0 = x0 * m4[..., 0] + x1 * m4[..., 1]
    r1 = x1 * m4[..., 3] + x0 * m4[..., 2]
    ref = np.stack([r0, r1], -1).reshape(batch, tokens, heads, dim).transpose(0, 2, 1, 3)
    assert np.array_equal(y, ref)
    # rotations keep each pair's norm
    n_in = np.hypot(x0, x1).transpose(0, 2, 1, 3)
    n_out = np.hypot(y[..., 0::2], y[..., 1::2])
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    # identity matrices only change the layout
    eye = rope_matrices(groups, tokens, dim, 20, identity=True)
    z = orc.model_aux(x, eye, None, 11, x.size, dim, channels=heads, spatial=tokens, groups=groups, batch=batch,
                      other_count=2 * dim * tokens * groups).reshape(batch, heads, tokens, dim)
    assert np.array_equal(z, x.transpose(0, 2, 1, 3))


@pytest.mark.parametrize("act", [0, 1])
def test_oracle_gated(orc, act):
    rows, width, channels = 6, 24, 56  # channels > 2*width: padded rows
    x = rng_normal((rows, channels), 21, 2.0)
    gate = x[:, :width] if act else x[:, width:2 * width]
    up = x[:, width:2 * width] if act else x[:, :width]
    y = orc.model_aux(x, None, None, 12, rows * width, width, channels=channels, spatial=rows, activation=act)
    np.testing.assert_allclose(y.reshape(rows, width), f64_act(gate, 5) * up, rtol=ACT_RTOL, atol=ACT_ATOL)
    attn_w = 5
    attn = rng_normal((rows, attn_w), 22)
    z = orc.model_aux(x, attn, None, 13, rows * (width + attn_w), width, channels=channels, spatial=rows,
                      groups=attn_w, other_count=rows * attn_w, activation=act).reshape(rows, width + attn_w)
    assert np.array_equal(z[:, :attn_w], attn)
    assert np.array_equal(z[:, attn_w:], y.reshape(rows, width))


# ---------------------------------------------------------------------------
# executor validation (CPU: every request fails before GPU work)
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def bufs():
    big = h.RpcBuffer(1 << 20)
    unmapped = h.RpcBuffer(4096, map_it=False)
    yield big, unmapped
    big.free()
    unmapped.free()


NONE = (-1, 0)


def aux_rc(out, inp, wgt, bias, **kw):
    args = dict(mode=0, count=64, width=16, channels=1, spatial=1, groups=1, batch=1, other_count=0, activation=0,
                eps=1e-6)
    args.update(kw)
    return h.execute(19, h.aux_params(out, inp, wgt, bias, **args))[0]


@pytest.mark.parametrize("size", [0, 75, 77, 80])
def test_aux_payload_size(size):
    payload = h.aux_params(NONE, NONE, NONE, NONE, 0, 64, 16, 1, 1, 1, 1, 0, 0, 0.0) + bytes(8)
    assert h.execute(19, payload[:size])[0] == -1


def test_aux_validation_codes(bufs):
    big, unmapped = bufs
    B = (big.fd, 0)
    bad = [
        dict(count=0), dict(mode=-1), dict(mode=14), dict(width=0), dict(channels=0), dict(spatial=0), dict(batch=0),
        dict(mode=8, count=63, width=8, spatial=8),
        dict(mode=2, groups=0), dict(mode=2, channels=6, groups=4),
        dict(mode=2, count=64, channels=8, groups=4, spatial=16),  # 8 x 16 values > count (checked here only)
        dict(mode=12, count=64, width=16, spatial=4, channels=31),
        dict(mode=12, count=64, width=16, spatial=4, channels=32, activation=2),
        dict(mode=12, count=60, width=16, spatial=4, channels=32),
        dict(mode=9, count=64, width=16, spatial=4, other_count=16, eps=-1.0),
        dict(mode=9, count=64, width=16, spatial=4, other_count=16, eps=float("nan")),
        dict(mode=9, count=64, width=16, spatial=4, other_count=17),
        dict(mode=10, count=64, width=16, spatial=4, other_count=20),
        dict(mode=11, count=64, width=15, spatial=4, other_count=120),
        dict(mode=11, count=64, width=16, spatial=4, other_count=100),
        dict(mode=11, count=128, width=16, spatial=4, batch=2, groups=3, other_count=128),
        dict(mode=3, count=64, other_count=0), dict(mode=3, count=64, other_count=5),
        dict(mode=13, count=64, width=12, spatial=4, groups=4, other_count=16, channels=24, activation=2),
        dict(mode=13, count=64, width=12, spatial=4, groups=4, other_count=15, channels=24),
        dict(mode=13, count=64, width=12, spatial=4, groups=4, other_count=16, channels=23),
    ]
    for kw in bad:
        wgt = B if kw.get("mode") in (3, 4, 9, 10, 11, 13) else NONE
        bias = B if kw.get("mode") in (9, 10) else NONE
        assert aux_rc(B, B, wgt, bias, **kw) == -1, kw
    # buffer presence rules
    assert aux_rc(B, B, NONE, NONE, mode=3, count=64, other_count=16) == -1       # mode 3 needs weights
    assert aux_rc(B, B, B, NONE, mode=9, count=64, width=16, spatial=4, other_count=16) == -1  # mode 9 needs bias
    assert aux_rc(B, B, B, NONE, mode=12, count=64, width=16, spatial=4, channels=32) == -1    # mode 12: none
    assert aux_rc(B, B, NONE, B, mode=11, count=64, width=16, spatial=4, other_count=128) == -1
    assert aux_rc(B, B, B, NONE, mode=0, count=64, width=16, other_count=15) == -1  # affine size != width
    # unmapped or missing tensors
    U = (unmapped.fd, 0)
    assert aux_rc(U, B, NONE, NONE) == -1
    assert aux_rc(B, U, NONE, NONE) == -1
    assert aux_rc(B, B, U, NONE, mode=3, count=64, other_count=16) == -1
    assert aux_rc(B, (999999, 0), NONE, NONE) == -1
    assert aux_rc((big.fd, (1 << 20) - 64), B, NONE, NONE) == -1  # output runs past the buffer
    # a norm with no whole row has no task (reference worker-pool code)
    assert aux_rc(B, B, NONE, NONE, mode=0, count=15, width=16) == -40


# ---------------------------------------------------------------------------
# GPU parity
# ---------------------------------------------------------------------------

def run_aux(hip, x, w, b, out_init=None, split=False, **kw):
    """hb_model_aux (or, with split, hb_model_aux_ws with its workspace)."""
    count = kw["count"]
    xd = hip.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    wd = None if w is None else hip.DeviceBuffer.from_array(np.ascontiguousarray(w, np.float32))
    bd = None if b is None else hip.DeviceBuffer.from_array(np.ascontiguousarray(b, np.float32))
    init = np.full(count, 3.5, np.float32) if out_init is None else out_init
    yd = hip.DeviceBuffer.from_array(init)
    ws = None
    if split:
        nbytes = hip.model_aux_workspace_bytes(kw["mode"], kw.get("channels", 1), kw.get("spatial", 1),
                                               kw.get("groups", 1), kw.get("batch", 1))
        assert nbytes > 0, kw
        ws = hip.DeviceBuffer(nbytes)
    hip.model_aux(yd, xd, wd, bd, workspace=ws, **kw)
    hip.sync()
    return yd.read(np.float32, count), init


NORM_CASES = [
    # mode, rows/groups shape, affine
    dict(mode=0, count=4096 * 3, width=4096, affine=True),
    dict(mode=0, count=1536 * 7 + 100, width=1536, affine=False),
    dict(mode=0, count=77 * 768, width=768, affine=True, activation=1),
    dict(mode=1, count=128 * 64, width=128, affine=True),
    dict(mode=1, count=33 * 5, width=33, affine=False),
    dict(mode=2, batch=2, channels=64, groups=32, spatial=37, affine=True),
    dict(mode=2, batch=1, channels=128, groups=32, spatial=4096, affine=False, activation=1),
    dict(mode=2, batch=1, channels=256, groups=32, spatial=16384, affine=True),  # 131072 per group: 3-pass kernel
    dict(mode=0, count=8192 * 20, width=8192, affine=True),                    # 8 float4 per thread
    dict(mode=1, count=2050 * 9, width=2050, affine=True),                     # width % 4 != 0
    dict(mode=9, batch=2, spatial=77, width=1536, per_batch=True),
    dict(mode=9, batch=1, spatial=300, width=3072, per_batch=False, activation=1),
    # two waves per row for 513-2048 values: 2, 3 and 4 float4 per thread
    dict(mode=1, count=2048 * 40, width=2048, affine=True),
    dict(mode=9, batch=2, spatial=50, width=2000, per_batch=True),
    dict(mode=0, count=1028 * 33, width=1028, affine=True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", NORM_CASES, ids=[f"m{c['mode']}_{i}" for i, c in enumerate(NORM_CASES)])
def test_aux_norms_gpu(hip, orc, case):
    c = dict(case)
    mode = c.pop("mode")
    act = c.pop("activation", 0)
    seed = 100 + mode
    if mode == 2:
        batch, channels, groups, spatial = c["batch"], c["channels"], c["groups"], c["spatial"]
        count, width = batch * channels * spatial, spatial
        w = rng_normal(channels, seed + 1) if c["affine"] else None
        b = rng_normal(channels, seed + 2) if c["affine"] else None
        kw = dict(mode=2, count=count, width=width, channels=channels, spatial=spatial, groups=groups, batch=batch,
                  other_count=channels if w is not None else 0, activation=act, eps=1e-5)
    elif mode == 9:
        batch, spatial, width = c["batch"], c["spatial"], c["width"]
        count = batch * spatial * width
        other = width * batch if c["per_batch"] else width
        w, b = rng_normal(other, seed + 1, 0.2), rng_normal(other, seed + 2, 0.2)
        kw = dict(mode=9, count=count, width=width, spatial=spatial, batch=batch, other_count=other, activation=act,
                  eps=1e-6)
    else:
        count, width = c["count"], c["width"]
        w = rng_normal(width, seed + 1) if c["affine"] else None
        b = rng_normal(width, seed + 2) if c["affine"] else None
        kw = dict(mode=mode, count=count, width=width, other_count=width if w is not None else 0, activation=act,
                  eps=1e-6)
    x = rng_normal(count, seed, 2.0) + 0.75
    got, init = run_aux(hip, x, w, b, **kw)
    want = orc.model_aux(x, w, b, out=init, **kw)
    rtol, atol = (ACT_RTOL, ACT_ATOL) if act else (NORM_RTOL, NORM_ATOL)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)
    # untouched tail (partial rows) keeps its contents
    covered = (count // kw["width"]) * kw["width"] if mode <= 1 else count
    assert (got[covered:] == init[covered:]).all()


@pytest.mark.gpu
@pytest.mark.parametrize("batch,channels,groups,spatial,affine,act,kind", [
    (1, 512, 32, 4096, True, 0, "normal"), (2, 128, 32, 16384, False, 1, "normal"),
    (1, 256, 32, 16388, True, 0, "normal"), (1, 64, 8, 65536 * 2, True, 0, "normal"),
    (1, 128, 32, 4096, True, 0, "offset"), (2, 64, 16, 8192, False, 0, "outlier"),
    (1, 256, 16, 4097, True, 0, "normal"),   # odd spatial: a quad spans two channels
    (1, 64, 8, 8192, True, 2, "normal")])    # affine then activation
def test_aux_group_norm_split_gpu(hip, orc, batch, channels, groups, spatial, affine, act, kind):
    """Group norm split over many workgroups per group (hb_model_aux_ws): the
    statistics come from sums shifted by each group's first value.  "offset"
    puts the mean far above the spread (1000 + 0.01 N(0, 1)), "outlier" makes
    every group's first value (the shift) 1e4 against values near 1."""
    count = batch * channels * spatial
    x = rng_normal(count, 150, 2.0) + 0.75
    if kind == "offset":
        x = (rng_normal(count, 153, 0.01) + 1000.0).astype(np.float32)
    elif kind == "outlier":
        x[::count // (batch * groups)] = 1e4
    w = rng_normal(channels, 151) if affine else None
    b = rng_normal(channels, 152) if affine else None
    kw = dict(mode=2, count=count, width=spatial, channels=channels, spatial=spatial, groups=groups, batch=batch,
              other_count=channels if affine else 0, activation=act, eps=1e-5)
    got, init = run_aux(hip, x, w, b, split=True, **kw)
    want = orc.model_aux(x, w, b, out=init, **kw)
    rtol, atol = (ACT_RTOL, ACT_ATOL) if act else (NORM_RTOL, NORM_ATOL)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [3, 4])
@pytest.mark.parametrize("count,other", [(1000, 10), (4096 * 1536, 1536), (12345, 12345)])
def test_aux_broadcast_gpu(hip, orc, mode, count, other):
    x, w = rng_normal(count, 200), rng_normal(other, 201)
    kw = dict(mode=mode, count=count, width=other, other_count=other)
    got, _ = run_aux(hip, x, w, None, **kw)
    assert np.array_equal(got, orc.model_aux(x, w, None, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [5, 6, 7])
def test_aux_activation_gpu(hip, orc, mode):
    x = rng_normal(100003, 300 + mode, 6.0)
    x[:6] = [0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30]
    kw = dict(mode=mode, count=x.size, width=1)
    got, _ = run_aux(hip, x, None, None, **kw)
    np.testing.assert_allclose(got, orc.model_aux(x, None, None, **kw), rtol=ACT_RTOL, atol=ACT_ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,width,spatial", [(1, 33, 65), (3, 512, 1024), (2, 7, 1)])
def test_aux_transpose_gpu(hip, orc, batch, width, spatial):
    x = rng_normal(batch * width * spatial, 400)
    kw = dict(mode=8, count=x.size, width=width, spatial=spatial, batch=batch)
    got, _ = run_aux(hip, x, None, None, **kw)
    assert np.array_equal(got, orc.model_aux(x, None, None, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("per_batch", [False, True])
def test_aux_modulation_gate_gpu(hip, orc, per_batch):
    batch, spatial, width = 2, 1024, 1536
    x = rng_normal(batch * spatial * width, 500)
    other = width * batch if per_batch else width
    w, b = rng_normal(other, 501), rng_normal(x.size, 502)
    kw = dict(mode=10, count=x.size, width=width, spatial=spatial, batch=batch, other_count=other)
    got, _ = run_aux(hip, x, w, b, **kw)
    assert np.array_equal(got, orc.model_aux(x, w, b, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("batch,tokens,heads,dim,groups", [(1, 4096, 24, 64, 1), (2, 77, 3, 128, 2), (1, 3, 1, 2, 1)])
def test_aux_rope_gpu(hip, orc, batch, tokens, heads, dim, groups):
    x = rng_normal(batch * tokens * heads * dim, 600)
    pe = rope_matrices(groups, tokens, dim, 601)
    kw = dict(mode=11, count=x.size, width=dim, channels=heads, spatial=tokens, groups=groups, batch=batch,
              other_count=2 * dim * tokens * groups)
    got, _ = run_aux(hip, x, pe, None, **kw)
    assert np.array_equal(got, orc.model_aux(x, pe, None, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("rows,width,channels", [(4096, 3072, 6144), (77, 100, 203)])
def test_aux_gated_gpu(hip, orc, act, rows, width, channels):
    x = rng_normal(rows * channels, 700 + act, 2.0)
    kw = dict(mode=12, count=rows * width, width=width, channels=channels, spatial=rows, activation=act)
    got, _ = run_aux(hip, x[:(rows - 1) * channels + 2 * width], None, None, **kw)
    want = orc.model_aux(x, None, None, **kw)
    np.testing.assert_allclose(got, want, rtol=ACT_RTOL, atol=ACT_ATOL)
    attn_w = 1536
    attn = rng_normal(rows * attn_w, 702)
    kw13 = dict(mode=13, count=rows * (width + attn_w), width=width, channels=channels, spatial=rows, groups=attn_w,
                other_count=rows * attn_w, activation=act)
    got13, _ = run_aux(hip, x, attn, None, **kw13)
    want13 = orc.model_aux(x, attn, None, **kw13)
    np.testing.assert_allclose(got13, want13, rtol=ACT_RTOL, atol=ACT_ATOL)


@pytest.mark.gpu
@pytest.mark.parametrize("device", [False, True])
def test_aux_opcode19_gpu(hip, orc, device):
    """The full opcode through execute_op_simple, host-resident and HBM-resident
    rpcmem tensors, including a partial last row that must keep its contents."""
    rows, width = 9, 1536
    count = rows * width + 50
    x = rng_normal(count, 800)
    w, b = rng_normal(width, 801), rng_normal(width, 802)
    bx, bw, bb, by = (h.RpcBuffer(a.nbytes, device=device) for a in (x, w, b, x))
    init = np.full(count, -2.0, np.float32)
    bx.write(x)
    bw.write(w)
    bb.write(b)
    by.write(init)
    rc, payload = h.execute(19, h.aux_params((by.fd, 0), (bx.fd, 0), (bw.fd, 0), (bb.fd, 0), 0, count, width, 1, 1, 1,
                                             1, width, 1, 1e-6))
    assert rc == 0
    got = by.read(np.float32, count)
    want = orc.model_aux(x, w, b, 0, count, width, other_count=width, activation=1, eps=1e-6, out=init)
    np.testing.assert_allclose(got, want, rtol=ACT_RTOL, atol=ACT_ATOL)
    assert (got[rows * width:] == -2.0).all()
    elapsed = np.frombuffer(payload[72:76], np.int32)[0]
    assert elapsed >= 0
    for buf in (bx, bw, bb, by):
        buf.free()
