"""Opcodes 8 / 10 / 11 / 12: fused QKV projection + RMS norm (+ RoPE) into
packed fp16 Q / K / V tiles.

CPU (the oracle and the boundary's argument checks):
  - the oracle's packed positions equal the readers of the reference's own
    test (src/host/test.c:854-884) and a model of the HVX instructions the
    reference packs with (wsf_to_vhf lane order, vscatter byte offsets,
    vshuff(-2) per the HVX shuffle algorithm; src/dsp/ops/mat_mul.c:1051-1125);
  - the magic-constant rsqrt is within 2 ulp of 1/sqrt;
  - the post-processing against float64 closed forms, and the reference's
    known-answer test (test.c:891-1060: its inputs, readers and 0.03 bound)
    run through the oracle;
  - execute_op_simple's codes for malformed requests (op_executor.cc:542-770,
    mat_mul.c:1373-1395, 1515-1583), which return before any GPU work.
GPU (marked): hb_qkv_post is bit-exact against oracle_qkv_post on the same
GEMM output; the four opcodes through execute_op_simple are bit-exact against
the oracle post-processing of the library's own F16 GEMM output, and within
the reference test's 0.03 of its float reference.
"""
import struct

import numpy as np
import pytest

import htp_ops as h

# ---------------------------------------------------------------- helpers ----


def ref_reader_index(which, tokens, head_dim, token, head, dim):
    """Halfword index of (token, head, dim) by the readers packed_q_value /
    packed_k_value / packed_v_value of the reference test (test.c:854-884)."""
    token_tiles = (tokens + 31) // 32
    head_elems = token_tiles * (head_dim // 32) * 1024
    if which == 2:
        tile = head * head_elems + ((dim // 32) * token_tiles + token // 32) * 1024
        return tile + ((token % 32) & ~1) * 32 + (dim % 32) * 2 + (token & 1)
    tile = head * head_elems + ((token // 32) * (head_dim // 32) + dim // 32) * 1024
    if which == 0:
        return tile + ((token % 32) & ~1) * 32 + (dim % 32) * 2 + (token & 1)
    return tile + ((dim % 32) & ~1) * 32 + (token % 32) * 2 + (dim & 1)


VB = 128  # HVX vector bytes


def hvx_vshuff(vu, vv, rt):
    """vshuff(Vu, Vv, Rt) on byte lists: the pair (v[0] = Vv, v[1] = Vu) with
    bytes k and k + offset swapped between the halves for each set bit of Rt,
    offsets ascending (the HVX vector shuffle).  Returns (lo, hi)."""
    hi, lo = list(vu), list(vv)
    off = 1
    while off < VB:
        if rt & off:
            for k in range(VB):
                if not k & off:
                    hi[k], lo[k + off] = lo[k + off], hi[k]
        off <<= 1
    return lo, hi


def model_pack_q(rows, n_rows, head_dim):
    """qkv_pack_q_tile (mat_mul.c:1051-1072): out_tile[r/2] = wsf_to_vhf(v1, v0),
    whose halfword lane 2i is v0[i] (row r) and 2i+1 is v1[i] (row r+1)."""
    out = [None] * (head_dim // 32 * 1024)
    for r in range(0, n_rows, 2):
        for d in range(head_dim // 32):
            v0 = [rows[r][32 * d + i] for i in range(32)]
            v1 = [rows[r + 1][32 * d + i] if r + 1 < n_rows else 0 for i in range(32)]
            vec = [None] * 64
            for i in range(32):
                vec[2 * i], vec[2 * i + 1] = v0[i], v1[i]
            base = d * 1024 + (r // 2) * 64
            out[base:base + 64] = vec
    return out


def model_pack_k(rows, n_rows, head_dim):
    """qkv_pack_k_tile (mat_mul.c:1078-1101): per row r and 64-column chunk d,
    vscatter of the 32 word lanes at byte offsets 128*i + 4*r of the chunk's
    two tiles (each word: columns 2i, 2i+1 of the chunk, low half first)."""
    buf = [None] * (head_dim * 32 * 2)  # bytes
    for r in range(n_rows):
        for d in range(head_dim // 64):
            for i in range(32):
                off = d * 4096 + 128 * i + 4 * r
                for b, c in enumerate((64 * d + 2 * i, 64 * d + 2 * i + 1)):
                    buf[off + 2 * b] = buf[off + 2 * b + 1] = rows[r][c]
    return [buf[2 * j] for j in range(len(buf) // 2)]


def model_pack_v(rows, head_dim, token_tile, token_tiles):
    """qkv_pack_v_tile (mat_mul.c:1103-1125): vshuff(row r+1, row r, -2) of
    each 64-column chunk, lo to column tile c/32 and hi to the next."""
    out = [None] * (token_tiles * head_dim // 32 * 1024)
    for r in range(0, 32, 2):
        for c in range(0, head_dim, 64):
            v0 = [x for j in range(64) for x in (rows[r][c + j],) * 2]  # byte lanes
            v1 = [x for j in range(64) for x in (rows[r + 1][c + j],) * 2]
            lo, hi = hvx_vshuff(v1, v0, -2)
            for t, vec in ((c // 32, lo), (c // 32 + 1, hi)):
                base = (t * token_tiles + token_tile) * 1024 + (r // 2) * 64
                out[base:base + 64] = vec[0::2]
    return out


def reference_case(n_heads, head_dim, input_dim, tokens, bias_kind, rope):
    """Inputs of the reference tests test_qkv_mul_channel (test.c:625-760,
    bias_kind "mul") and test_qkv_rope_channel (test.c:891-975, bias_kind
    "rope" or "none")."""
    cols = 3 * n_heads * head_dim
    t = np.arange(tokens)[:, None]
    c = np.arange(input_dim)[None, :]
    act = ((((t * 11 + c * 5) % 37) - 18).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    r = np.arange(input_dim)[:, None]
    cc = np.arange(cols)[None, :]
    w = ((((r * 13 + cc * 7) % 101) - 50).astype(np.float32) * np.float32(0.001)).astype(np.float32)
    ci = np.arange(cols)
    if bias_kind == "mul":
        bias = (((ci % 17) - 8).astype(np.float32) * np.float32(0.01)).astype(np.float32)
        d = np.arange(head_dim)
        qn = (np.float32(1.0) + (d % 7).astype(np.float32) * np.float32(0.01)).astype(np.float32)
        kn = (np.float32(1.0) - (d % 5).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    else:
        bias = np.zeros(cols, np.float32) if bias_kind == "none" else \
            (((ci % 19) - 9).astype(np.float32) * np.float32(0.007)).astype(np.float32)
        d = np.arange(head_dim)
        qn = (np.float32(0.9) + (d % 11).astype(np.float32) * np.float32(0.013)).astype(np.float32)
        kn = (np.float32(1.1) - (d % 7).astype(np.float32) * np.float32(0.009)).astype(np.float32)
    pe = None
    if rope:
        tt = np.arange(tokens, dtype=np.float32)[:, None]
        dd = np.arange(head_dim // 2, dtype=np.float32)[None, :]
        ang = (np.float32(0.013) * (tt + 1) * (dd + 1)).astype(np.float32)
        pe = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], axis=-1).astype(np.float32).ravel()
    return act, w, bias, qn, kn, pe


def hmx_raw(act, w):
    """GEMM output as the HMX path forms it: fp16 activations and weights,
    an exact dot product, one fp16 rounding (mat_mul.c:1297-1330)."""
    a = act.astype(np.float16).astype(np.float64)
    b = w.astype(np.float16).astype(np.float64)
    return (a @ b).astype(np.float16).astype(np.float32)


def float_reference(act, w, bias, qn, kn, pe, n_heads, head_dim, rope):
    """The reference test's float expectation (test.c:1005-1050), in float64:
    [3][tokens][n_heads][head_dim]."""
    raw = act.astype(np.float64) @ w.astype(np.float64) + bias.astype(np.float64)
    tokens = act.shape[0]
    raw = raw.reshape(tokens, 3, n_heads, head_dim)
    q, k, v = raw[:, 0], raw[:, 1], raw[:, 2]
    out = []
    for x, g in ((q, qn), (k, kn)):
        inv = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / head_dim + 1e-6)
        y = x * inv * g.astype(np.float64)
        if rope:
            m = pe.reshape(tokens, 1, head_dim // 2, 4).astype(np.float64)
            x0, x1 = y[..., 0::2], y[..., 1::2]
            y = y.copy()
            y[..., 0::2] = x0 * m[..., 0] + x1 * m[..., 1]
            y[..., 1::2] = x0 * m[..., 2] + x1 * m[..., 3]
        out.append(y)
    out.append(v)
    return out


def unpack(packed_bits, which, tokens, n_heads, head_dim):
    """Packed fp16 bits -> float32 [tokens][n_heads][head_dim] via the reference readers."""
    t = np.arange(tokens)[:, None, None]
    hh = np.arange(n_heads)[None, :, None]
    d = np.arange(head_dim)[None, None, :]
    idx = ref_reader_index(which, tokens, head_dim, t, hh, d)
    return packed_bits.view(np.float16)[idx].astype(np.float32)


def max_errors(q, k, v, expected, tokens, n_heads, head_dim):
    errs = []
    for which, got in enumerate((q, k, v)):
        e = expected[which].astype(np.float32).astype(np.float16).astype(np.float64)
        errs.append(float(np.abs(unpack(got, which, tokens, n_heads, head_dim) - e).max()))
    return errs


# ----------------------------------------------------------- CPU: layout -----


@pytest.mark.parametrize("head_dim,tokens", [(64, 32), (128, 45), (64, 70)])
def test_index_matches_reference_readers(orc, head_dim, tokens):
    tiles = (tokens + 31) // 32
    elems = orc.qkv_head_elems(tiles, head_dim)
    for which in range(3):
        seen = np.zeros(elems, np.int32)
        for t in range(tiles * 32):
            for c in range(head_dim):
                i = orc.qkv_index(which, tiles, head_dim, t // 32, t % 32, c)
                seen[i] += 1
                if t < tokens:
                    assert i == ref_reader_index(which, tokens, head_dim, t, 0, c), (which, t, c)
        assert (seen == 1).all(), which  # a bijection onto the head's region


@pytest.mark.parametrize("head_dim", [64, 128])
def test_index_matches_hvx_instruction_model(orc, head_dim):
    n_rows, tiles, tt = 32, 2, 1
    rows = [[(r, c) for c in range(head_dim)] for r in range(n_rows)]
    q = model_pack_q(rows, n_rows, head_dim)
    k = model_pack_k(rows, n_rows, head_dim)
    v = model_pack_v(rows, head_dim, tt, tiles)
    for r in range(n_rows):
        for c in range(head_dim):
            iq = orc.qkv_index(0, tiles, head_dim, tt, r, c) - tt * head_dim * 32
            ik = orc.qkv_index(1, tiles, head_dim, tt, r, c) - tt * head_dim * 32
            assert q[iq] == (r, c) and k[ik] == (r, c), (r, c)
            assert v[orc.qkv_index(2, tiles, head_dim, tt, r, c)] == (r, c), (r, c)


def test_hvx_vshuff_model_interleaves_halfwords():
    a = list(range(VB))
    b = list(range(1000, 1000 + VB))
    lo, hi = hvx_vshuff(b, a, -2)
    assert lo[:8] == [0, 1, 1000, 1001, 2, 3, 1002, 1003]
    assert hi[:4] == [64, 65, 1064, 1065]


def test_partial_rows_in_hvx_model_are_zero(orc):
    rows = [[(r, c) for c in range(64)] for r in range(5)]
    q = model_pack_q(rows, 5, 64)
    assert q[orc.qkv_index(0, 1, 64, 0, 5, 3)] == 0  # row 5 of the pair (4, 5) is the zero vector


# ------------------------------------------------------------ CPU: rsqrt -----


def test_rsqrt_within_two_ulp(orc):
    rng = np.random.default_rng(5)
    xs = np.concatenate([np.float32(2.0) ** rng.uniform(-120, 120, 4000), rng.uniform(1e-6, 4.0, 2000)])
    for x in xs.astype(np.float32):
        y = np.float32(orc.qkv_rsqrt(float(x)))
        exact = 1.0 / np.sqrt(np.float64(x))
        assert abs(np.float64(y) - exact) <= 2 * np.spacing(np.float32(exact)), x


def test_rsqrt_is_three_newton_steps_from_the_magic_start(orc):
    for x in (np.float32(1.0), np.float32(0.37), np.float32(123.5)):
        y = (np.uint32(0x5F3759DF) - (np.float32(x).view(np.uint32) >> np.uint32(1))).view(np.float32)
        half = np.float32(x) * np.float32(0.5)
        for _ in range(3):
            y = np.float32(y * np.float32(np.float32(1.5) - np.float32(half * np.float32(y * y))))
        assert np.float32(orc.qkv_rsqrt(float(x))) == y


# ------------------------------------------------------------- CPU: post -----


def post_inputs(tokens, n_heads, head_dim, seed, rope_tokens=0):
    rng = np.random.default_rng(seed)
    cols = 3 * n_heads * head_dim
    raw = rng.normal(0, 1.5, (tokens, cols)).astype(np.float16).astype(np.float32)
    bias = rng.normal(0, 0.2, cols).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, head_dim).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, head_dim).astype(np.float32)
    pe = None
    if rope_tokens:
        ang = rng.uniform(-np.pi, np.pi, (rope_tokens, head_dim // 2))
        pe = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).astype(np.float32).ravel()
    return raw, bias, qn, kn, pe


@pytest.mark.parametrize("head_dim", [64, 128])
def test_post_normalized_rows_and_v(orc, head_dim):
    tokens, n_heads = 45, 2
    raw, bias, _, _, _ = post_inputs(tokens, n_heads, head_dim, 3)
    ones = np.ones(head_dim, np.float32)
    tiles = 2
    q, k, v = orc.qkv_post(raw, bias, ones, ones, None, 0, 0, tokens, n_heads, head_dim, tiles)
    x = (raw.astype(np.float64) + bias.astype(np.float32)).reshape(tokens, 3, n_heads, head_dim)
    for which, got in ((0, q), (1, k)):
        y = unpack(got, which, tokens, n_heads, head_dim).astype(np.float64)
        rms = np.sqrt((y * y).mean(-1))
        assert np.abs(rms - 1).max() < 2e-3  # fp16 rounding of each element
        ref = x[:, which] / np.sqrt((x[:, which] ** 2).mean(-1, keepdims=True) + 1e-6)
        assert np.abs(y - ref).max() <= 2.0 ** -10 * np.abs(ref).max() * 1.01
    # V is fp16(raw + bias), exactly
    vv = unpack(v, 2, tokens, n_heads, head_dim)
    exp_v = (raw + np.tile(bias, (tokens, 1))).reshape(tokens, 3, n_heads, head_dim)[:, 2].astype(np.float16)
    assert np.array_equal(vv.astype(np.float16).view(np.uint16), exp_v.view(np.uint16))
    # padded rows 45..63 of the last tile are zeros
    for which, got in ((0, q), (1, k), (2, v)):
        for r in range(tokens, 64):
            for c in (0, head_dim - 1):
                assert got[orc.qkv_index(which, tiles, head_dim, r // 32, r % 32, c)] == 0


def test_post_bias_none_equals_zero_bias(orc):
    raw, bias, qn, kn, _ = post_inputs(33, 2, 64, 4)
    a = orc.qkv_post(raw, None, qn, kn, None, 0, 0, 33, 2, 64, 2)
    b = orc.qkv_post(raw, np.zeros_like(bias), qn, kn, None, 0, 0, 33, 2, 64, 2)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_post_gamma_scales_columns(orc):
    raw, bias, qn, kn, _ = post_inputs(32, 1, 64, 6)
    ones = np.ones(64, np.float32)
    q1, k1, _ = orc.qkv_post(raw, bias, ones, ones, None, 0, 0, 32, 1, 64, 1)
    q2, k2, _ = orc.qkv_post(raw, bias, qn, kn, None, 0, 0, 32, 1, 64, 1)
    for w, a, b, g in ((0, q1, q2, qn), (1, k1, k2, kn)):
        ya = unpack(a, w, 32, 1, 64).astype(np.float64) * g
        yb = unpack(b, w, 32, 1, 64).astype(np.float64)
        assert np.abs(ya - yb).max() <= 2.0 ** -9 * np.abs(yb).max()


def test_post_identity_rotation_and_pair_norms(orc):
    tokens, n_heads, hd = 40, 2, 128
    raw, bias, qn, kn, pe = post_inputs(tokens, n_heads, hd, 7, rope_tokens=tokens)
    ident = np.tile(np.array([1, 0, 0, 1], np.float32), tokens * hd // 2)
    plain = orc.qkv_post(raw, bias, qn, kn, None, 0, 0, tokens, n_heads, hd, 2)
    same = orc.qkv_post(raw, bias, qn, kn, ident, 0, tokens, tokens, n_heads, hd, 2)
    for x, y in zip(plain, same):
        assert np.array_equal(x, y)
    rot = orc.qkv_post(raw, bias, qn, kn, pe, 0, tokens, tokens, n_heads, hd, 2)
    for w in (0, 1):
        a = unpack(plain[w], w, tokens, n_heads, hd).astype(np.float64)
        b = unpack(rot[w], w, tokens, n_heads, hd).astype(np.float64)
        na = np.hypot(a[..., 0::2], a[..., 1::2])
        nb = np.hypot(b[..., 0::2], b[..., 1::2])
        assert np.abs(na - nb).max() <= 2.0 ** -9 * na.max()
        assert not np.array_equal(a, b)
    assert np.array_equal(plain[2], rot[2])  # V is never rotated


def test_post_rope_offset_and_count(orc):
    """Row r of a call uses matrix rope_offset + r and stops at rope_count
    (mat_mul.c:1210-1231, the token of :1343-1345)."""
    tokens, hd = 32, 64
    raw, bias, qn, kn, pe = post_inputs(tokens, 1, hd, 8, rope_tokens=50)
    full = orc.qkv_post(raw, bias, qn, kn, pe[10 * hd * 2:], 0, 40, tokens, 1, hd, 1)
    off = orc.qkv_post(raw, bias, qn, kn, pe, 10, 50, tokens, 1, hd, 1)
    for x, y in zip(full, off):
        assert np.array_equal(x, y)
    cut = orc.qkv_post(raw, bias, qn, kn, pe, 10, 25, tokens, 1, hd, 1)
    plain = orc.qkv_post(raw, bias, qn, kn, None, 0, 0, tokens, 1, hd, 1)
    a, b, c = (unpack(x[0], 0, tokens, 1, hd) for x in (off, cut, plain))
    assert np.array_equal(b[:15], a[:15]) and np.array_equal(b[15:], c[15:])
    # a negative offset or a zero count disables the rotation
    for o, n in ((-1, 50), (0, 0)):
        z = orc.qkv_post(raw, bias, qn, kn, pe, o, n, tokens, 1, hd, 1)
        assert np.array_equal(z[0], plain[0])


def test_post_output_offset_keeps_other_tiles(orc):
    raw, bias, qn, kn, _ = post_inputs(20, 1, 64, 9)
    raw2, _, _, _, _ = post_inputs(32, 1, 64, 10)
    q, k, v = orc.qkv_post(raw2, bias, qn, kn, None, 0, 0, 32, 1, 64, 3)
    q, k, v = orc.qkv_post(raw, bias, qn, kn, None, 0, 0, 20, 1, 64, 3, out_offset=64, out=(q, k, v))
    alone = orc.qkv_post(raw, bias, qn, kn, None, 0, 0, 20, 1, 64, 1)
    for which, (got, one) in enumerate(zip((q, k, v), alone)):
        for r in range(32):
            for c in range(0, 64, 7):
                assert got[orc.qkv_index(which, 3, 64, 2, r, c)] == one[orc.qkv_index(which, 1, 64, 0, r, c)]
        assert got[orc.qkv_index(which, 3, 64, 0, 3, 5)] != 0  # the first call's tile stays


@pytest.mark.parametrize("bias_kind", ["rope", "none"])
def test_reference_known_answer_through_the_oracle(orc, bias_kind):
    """test_qkv_rope_channel (test.c:891-1060) on the CPU: 24 heads x 128,
    input 1536, 64 tokens, its inputs and its 0.03 bound on every element."""
    n_heads, hd, k, tokens = 24, 128, 1536, 64
    act, w, bias, qn, kn, pe = reference_case(n_heads, hd, k, tokens, bias_kind, rope=True)
    raw = hmx_raw(act, w)
    tiles = 2
    q, kk, v = orc.qkv_post(raw, bias, qn, kn, pe, 0, tokens, tokens, n_heads, hd, tiles)
    expected = float_reference(act, w, bias, qn, kn, pe, n_heads, hd, rope=True)
    errs = max_errors(q, kk, v, expected, tokens, n_heads, hd)
    assert max(errs) <= 0.03, errs
    # the dual request of the same test: image rows 0..31, text rows 32..63
    # at rotary offsets 0 and 32, one output (op_executor.cc:707-770)
    out = orc.qkv_post(raw[:32], bias, qn, kn, pe, 0, tokens, 32, n_heads, hd, tiles)
    out = orc.qkv_post(raw[32:], bias, qn, kn, pe, 32, tokens, 32, n_heads, hd, tiles, out_offset=32, out=out)
    for x, y in zip(out, (q, kk, v)):
        assert np.array_equal(x, y)


def test_reference_opcode8_known_answer_through_the_oracle(orc):
    """test_qkv_mul_channel (test.c:625-820): token 0 of head 0, 0.01 bound."""
    n_heads, hd, k, tokens = 24, 64, 1536, 32
    act, w, bias, qn, kn, _ = reference_case(n_heads, hd, k, tokens, "mul", rope=False)
    q, kk, v = orc.qkv_post(hmx_raw(act, w), bias, qn, kn, None, 0, 0, tokens, n_heads, hd, 1)
    e = float_reference(act, w, bias, qn, kn, None, n_heads, hd, rope=False)
    f = lambda bits, i: float(bits[i:i + 1].view(np.float16)[0])
    assert abs(f(q, 0) - e[0][0, 0, 0]) < 0.01
    assert abs(f(kk, 0) - e[1][0, 0, 0]) < 0.01 and abs(f(kk, 1) - e[1][0, 0, 1]) < 0.01
    assert abs(f(v, 0) - e[2][0, 0, 0]) < 0.01 and abs(f(v, 2) - e[2][0, 0, 1]) < 0.01


# --------------------------------------------------- CPU: request validation --

HD, HEADS, KDIM, TOK = 64, 24, 64, 32
QKV_BYTES = HEADS * 1 * (HD // 32) * 1024 * 2
W_BYTES = KDIM * 3 * HEADS * HD * 2
OFF = {"q": 0, "k": QKV_BYTES, "v": 2 * QKV_BYTES, "act": 3 * QKV_BYTES, "w": 3 * QKV_BYTES + TOK * KDIM * 4}
OFF["bias"] = OFF["w"] + W_BYTES
OFF["qn"] = OFF["bias"] + 3 * HEADS * HD * 4
OFF["kn"] = OFF["qn"] + 512
OFF["pe"] = OFF["kn"] + 512
TOTAL = OFF["pe"] + 2 * TOK * HD * 2 * 4


@pytest.fixture(scope="module")
def qbufs():
    big = h.RpcBuffer(TOTAL + 4096)
    unmapped = h.RpcBuffer(4096, map_it=False)
    yield big, unmapped
    for b in (big, unmapped):
        b.free()


def single(big, tokens=TOK, input_dim=KDIM, heads=HEADS, hd=HD, **over):
    a = {n: (big.fd, o) for n, o in OFF.items()}
    a.update(over)
    return h.qkv_params(a["q"], a["k"], a["v"], a["act"], a["w"], a["bias"], a["qn"], a["kn"], tokens, input_dim,
                        heads, hd)


def rope1(big, tokens=TOK, offset=0, count=TOK, heads=HEADS, hd=HD, **over):
    a = {n: (big.fd, o) for n, o in OFF.items()}
    a.update(over)
    return h.qkv_rope_params(a["q"], a["k"], a["v"], a["act"], a["w"], a["bias"], a["qn"], a["kn"], a["pe"], tokens,
                             KDIM, heads, hd, offset, count)


def dual(big, image=32, text=1, heads=HEADS, hd=HD, rope=False, io=0, to=0, **over):
    a = {n: (big.fd, o) for n, o in OFF.items()}
    a.update(over)
    part = (a["act"], a["w"], a["bias"], a["qn"], a["kn"])
    text_part = (a.get("tact", a["act"]), a["w"], a.get("tbias", a["bias"]), a["qn"], a["kn"])
    if rope:
        return h.qkv_dual_rope_params(a["q"], a["k"], a["v"], part, text_part, a["pe"], image, text, KDIM, heads, hd,
                                      io, to)
    return h.qkv_dual_params(a["q"], a["k"], a["v"], part, text_part, image, text, KDIM, heads, hd)


def test_qkv_payload_sizes(qbufs):
    big = qbufs[0]
    for op, p in ((8, single(big)), (11, rope1(big)), (10, dual(big)), (12, dual(big, rope=True))):
        assert h.execute(op, p[:-1])[0] == -1, op
        assert h.execute(op, b"")[0] == -1, op


@pytest.mark.parametrize("heads,hd", [(16, 64), (24, 32), (24, 256), (38, 128), (0, 64), (-24, 64)])
def test_qkv_unsupported_shapes(qbufs, heads, hd):
    big = qbufs[0]
    for op, p in ((8, single(big, heads=heads, hd=hd)), (11, rope1(big, heads=heads, hd=hd)),
                  (10, dual(big, heads=heads, hd=hd)), (12, dual(big, heads=heads, hd=hd, rope=True))):
        assert h.execute(op, p)[0] == -1, (op, heads, hd)


def test_qkv_dimension_codes(qbufs):
    big = qbufs[0]
    assert h.execute(8, single(big, tokens=0))[0] == -1
    assert h.execute(8, single(big, input_dim=48))[0] == -1
    assert h.execute(8, single(big, input_dim=0))[0] == -1
    assert h.execute(11, rope1(big, offset=-1))[0] == -1
    assert h.execute(11, rope1(big, count=0))[0] == -1
    for image, text in ((0, 4), (31, 4), (32, 0), (32, -1), (-32, 4)):
        assert h.execute(10, dual(big, image=image, text=text))[0] == -1, (image, text)
        assert h.execute(12, dual(big, image=image, text=text, rope=True))[0] == -1, (image, text)
    assert h.execute(12, dual(big, rope=True, io=-1))[0] == -1
    assert h.execute(12, dual(big, rope=True, to=-1))[0] == -1


def test_qkv_unmapped_and_misaligned(qbufs):
    big, unmapped = qbufs
    for name in ("q", "k", "v", "act", "w", "bias", "qn", "kn"):
        assert h.execute(8, single(big, **{name: (unmapped.fd, 0)}))[0] == -1, name
    for name in ("q", "k", "v", "act", "w"):
        assert h.execute(8, single(big, **{name: (big.fd, OFF[name] + 64)}))[0] == -1, name
        assert h.execute(11, rope1(big, **{name: (big.fd, OFF[name] + 64)}))[0] == -1, name
        assert h.execute(10, dual(big, **{name: (big.fd, OFF[name] + 64)}))[0] == -1, name
    assert h.execute(10, dual(big, tact=(big.fd, OFF["act"] + 64)))[0] == -1
    assert h.execute(10, dual(big, tact=(unmapped.fd, 0)))[0] == -1
    # opcode 8 needs its bias; 10/11/12 take fd < 0 as none, but a named
    # buffer that is not mapped is still an error
    assert h.execute(8, single(big, bias=(-1, 0)))[0] == -1
    assert h.execute(11, rope1(big, bias=(unmapped.fd, 0)))[0] == -1
    assert h.execute(10, dual(big, tbias=(unmapped.fd, 0)))[0] == -1


def test_qkv_out_of_range_buffers(qbufs):
    big = qbufs[0]
    end = big.nbytes
    assert h.execute(8, single(big, q=(big.fd, end - 128)))[0] == -1
    assert h.execute(8, single(big, w=(big.fd, end - 1024)))[0] == -1


def test_qkv_rejected_requests_write_nothing(qbufs):
    big = qbufs[0]
    big.write(np.full(64, 0x5A, np.uint8), OFF["q"])
    p = single(big, input_dim=48)
    rc, after = h.execute(8, p)
    assert rc == -1 and after == p
    assert (big.read(np.uint8, 64, OFF["q"]) == 0x5A).all()


# ------------------------------------------------------------------- GPU -----


def dev(arr):
    return h.DeviceBuffer.from_array(np.ascontiguousarray(arr))


@pytest.mark.gpu
@pytest.mark.parametrize("tokens,n_heads,hd,rope,bias,offset,count,out_tile", [
    (32, 2, 64, False, True, 0, 0, 0),
    (45, 3, 128, True, True, 0, 45, 0),     # ragged last tile
    (70, 2, 64, True, False, 5, 60, 1),     # rotary offset, rows past the count, later output tiles
    (1, 1, 128, True, True, 3, 4, 0),       # one token
    (64, 24, 128, True, True, 0, 64, 0),    # the reference test's shape
    (96, 38, 64, False, True, 0, 0, 0),
])
def test_hb_qkv_post_bit_exact(hip, orc, tokens, n_heads, hd, rope, bias, offset, count, out_tile):
    raw, b, qn, kn, pe = post_inputs(tokens, n_heads, hd, tokens + hd, rope_tokens=offset + tokens + 3 if rope else 0)
    b = b if bias else None
    tiles = out_tile + (tokens + 31) // 32
    size = n_heads * orc.qkv_head_elems(tiles, hd)
    ref = orc.qkv_post(raw, b, qn, kn, pe, offset, count, tokens, n_heads, hd, tiles, out_offset=32 * out_tile,
                       out=tuple(np.full(size, 0x1234, np.uint16) for _ in range(3)))
    outs = [dev(np.full(size, 0x1234, np.uint16)) for _ in range(3)]
    h.qkv_post(*outs, dev(raw), dev(b) if bias else None, dev(qn), dev(kn), dev(pe) if rope else None, offset, count,
               tokens, n_heads, hd, tiles, 32 * out_tile)
    h.sync()
    for which, (o, r) in enumerate(zip(outs, ref)):
        got = o.read(np.uint16, size)
        assert np.array_equal(got, r), (which, int((got != r).sum()))


@pytest.mark.gpu
def test_hb_qkv_post_rejects_bad_arguments(hip):
    x = h.DeviceBuffer(1 << 16)
    base = (x, x, x, x, None, x, x, None)
    with pytest.raises(h.HtpOpsError):
        h.qkv_post(*base, 0, 0, 32, 1, 96, 1)          # head_dim
    with pytest.raises(h.HtpOpsError):
        h.qkv_post(*base, 0, 0, 33, 1, 64, 1)          # tokens past the output tiles
    with pytest.raises(h.HtpOpsError):
        h.qkv_post(*base, 0, 0, 32, 1, 64, 2, 16)      # offset not a tile


def gpu_case(orc, op, bias_kind, device, shape=None):
    """The reference test's request for op (24 heads; 8: head_dim 64,
    32 tokens; 10/11/12: head_dim 128, 64 tokens; `shape` = (heads, head_dim)
    overrides, as the test's HTP_QKV_ROPE_HEADS / _HEAD_DIM do), laid out in
    one buffer."""
    rope = op in (11, 12)
    n_heads, hd, k, tokens = (24, 64, 1536, 32) if op == 8 else (24, 128, 1536, 64)
    if shape is not None:
        n_heads, hd = shape
    act, w, bias, qn, kn, pe = reference_case(n_heads, hd, k, tokens, bias_kind, rope)
    tiles = (tokens + 31) // 32
    qkv_bytes = n_heads * orc.qkv_head_elems(tiles, hd) * 2
    align = lambda x: (x + 127) // 128 * 128
    offs, pos = {}, 0
    for name, nbytes in (("act", act.nbytes), ("w", w.size * 2), ("bias", bias.nbytes), ("qn", qn.nbytes),
                         ("kn", kn.nbytes), ("pe", 0 if pe is None else pe.nbytes), ("q", qkv_bytes),
                         ("k", qkv_bytes), ("v", qkv_bytes)):
        offs[name] = pos
        pos = align(pos + nbytes)
    buf = h.RpcBuffer(pos, device=device)
    permuted = h.permute_f16(w.astype(np.float16).view(np.uint16))
    for name, arr in (("act", act), ("w", permuted), ("bias", bias), ("qn", qn), ("kn", kn), ("pe", pe)):
        if arr is not None:
            buf.write(arr, offs[name])
    for name in ("q", "k", "v"):
        buf.write(np.zeros(qkv_bytes, np.uint8), offs[name])
    a = {n: (buf.fd, o) for n, o in offs.items()}
    b = (-1, 0) if bias_kind == "none" else a["bias"]
    if op == 8:
        p = h.qkv_params(a["q"], a["k"], a["v"], a["act"], a["w"], b, a["qn"], a["kn"], tokens, k, n_heads, hd)
    elif op == 11:
        p = h.qkv_rope_params(a["q"], a["k"], a["v"], a["act"], a["w"], b, a["qn"], a["kn"], a["pe"], tokens, k,
                              n_heads, hd, 0, tokens)
    else:
        text_act = (buf.fd, offs["act"] + 32 * k * 4)
        img = (a["act"], a["w"], b, a["qn"], a["kn"])
        txt = (text_act, a["w"], b, a["qn"], a["kn"])
        if op == 10:
            p = h.qkv_dual_params(a["q"], a["k"], a["v"], img, txt, 32, 32, k, n_heads, hd)
        else:
            p = h.qkv_dual_rope_params(a["q"], a["k"], a["v"], img, txt, a["pe"], 32, 32, k, n_heads, hd, 0, 32)
    return dict(buf=buf, offs=offs, payload=p, act=act, w=w, permuted=permuted, bias=bias, qn=qn, kn=kn, pe=pe,
                n_heads=n_heads, hd=hd, k=k, tokens=tokens, tiles=tiles, qkv_bytes=qkv_bytes, rope=rope)


def library_raw(c, parts=None):
    """The library's own F16 GEMM output for the case (mode 0, no bias), one
    call per part of `parts` rows (the executor multiplies each part of a
    dual request on its own, and the kernel a call takes depends on its row
    count)."""
    m, k, n = c["tokens"], c["k"], 3 * c["n_heads"] * c["hd"]
    packed = h.f16_prepack(dev(c["permuted"]), k, n)
    out = []
    for r0, r1 in (parts or [(0, m)]):
        rows = r1 - r0
        y = h.DeviceBuffer(rows * n * 4)
        ws = h.DeviceBuffer(max(h.f16_workspace_bytes(rows, k, n), 1))
        h.f16_gemm(y, dev(np.ascontiguousarray(c["act"][r0:r1])), packed, None, rows, k, n, n, 0, workspace=ws)
        h.sync()
        out.append(y.read(np.float32, rows * n).reshape(rows, n))
    return np.concatenate(out)


@pytest.mark.gpu
@pytest.mark.parametrize("op,bias_kind,device,shape", [
    (8, "mul", False, None), (8, "mul", True, None),
    (10, "rope", True, None), (10, "none", False, None),
    (11, "rope", False, None), (11, "none", True, None),
    (12, "rope", True, None), (12, "none", False, None),
    # every supported head shape (op_reg.h:23-39): 24 / 30 heads of 64 or 128, 38 heads of 64
    (11, "rope", True, (30, 128)), (12, "rope", True, (30, 64)), (11, "rope", True, (38, 64)),
    (12, "none", True, (24, 64)), (8, "mul", True, (38, 64)), (10, "rope", True, (30, 128)),
])
def test_qkv_opcodes_end_to_end(hip, orc, op, bias_kind, device, shape):
    c = gpu_case(orc, op, bias_kind, device, shape)
    rc, after = h.execute(op, c["payload"])
    assert rc == 0, h.last_error()
    elapsed = struct.unpack_from("<i", after, len(after) - 4)[0]
    assert elapsed >= 0
    got = [c["buf"].read(np.uint16, c["qkv_bytes"] // 2, c["offs"][n]) for n in ("q", "k", "v")]
    # bit-exact: the oracle's post-processing of the library's GEMM output
    raw = library_raw(c, [(0, 32), (32, c["tokens"])] if op in (10, 12) else None)
    bias = None if bias_kind == "none" else c["bias"]
    t, nh, hd, tiles = c["tokens"], c["n_heads"], c["hd"], c["tiles"]
    if op in (10, 12):
        rope_off = (0, 32) if op == 12 else (0, 0)
        ref = orc.qkv_post(raw[:32], bias, c["qn"], c["kn"], c["pe"], rope_off[0], t, 32, nh, hd, tiles)
        ref = orc.qkv_post(raw[32:], bias, c["qn"], c["kn"], c["pe"], rope_off[1], t, 32, nh, hd, tiles,
                           out_offset=32, out=ref)
    else:
        ref = orc.qkv_post(raw, bias, c["qn"], c["kn"], c["pe"], 0, t if c["rope"] else 0, t, nh, hd, tiles)
    for which in range(3):
        assert np.array_equal(got[which], ref[which]), (which, int((got[which] != ref[which]).sum()))
    # and the reference test's own bound against its float expectation
    b = np.zeros_like(c["bias"]) if bias is None else bias
    expected = float_reference(c["act"], c["w"], b, c["qn"], c["kn"], c["pe"], nh, hd, c["rope"])
    errs = max_errors(*got, expected, t, nh, hd)
    assert max(errs) <= (0.01 if op == 8 else 0.03), errs


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads,hd,image,text", [
    (30, 64, 64, 45),     # both parts: GEMM, then the post-processing kernel
    (24, 64, 256, 1100),  # text part: the GEMM with the post-processing in its epilogue
    (24, 128, 96, 600),   # the same with heads of 128
])
def test_qkv_ragged_dual_and_rotary_window(hip, orc, n_heads, hd, image, text):
    """Dual request with a ragged text part (input 256) and rotary offsets
    3 / 70, against the oracle post-processing of the library's GEMM."""
    k = 256
    tokens = image + text
    tiles = (tokens + 31) // 32
    rng = np.random.default_rng(11)
    cols = 3 * n_heads * hd
    act = rng.normal(0, 1, (tokens, k)).astype(np.float32)
    w_img = rng.normal(0, 0.05, (k, cols)).astype(np.float16)
    w_txt = rng.normal(0, 0.05, (k, cols)).astype(np.float16)
    bias = rng.normal(0, 0.1, cols).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    rope_tokens = max(3 + image, 70 + text)
    ang = rng.uniform(-3, 3, (rope_tokens, hd // 2))
    pe = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).astype(np.float32).ravel()
    qkv_bytes = n_heads * orc.qkv_head_elems(tiles, hd) * 2
    pieces = [("act", act), ("wi", h.permute_f16(w_img.view(np.uint16))), ("wt", h.permute_f16(w_txt.view(np.uint16))),
              ("bias", bias), ("qn", qn), ("kn", kn), ("pe", pe)]
    offs, pos = {}, 0
    for name, arr in pieces:
        offs[name] = pos
        pos = (pos + arr.nbytes + 127) // 128 * 128
    for name in ("q", "k", "v"):
        offs[name] = pos
        pos += qkv_bytes
    buf = h.RpcBuffer(pos, device=True)
    for name, arr in pieces:
        buf.write(arr, offs[name])
    a = {n: (buf.fd, o) for n, o in offs.items()}
    img = (a["act"], a["wi"], a["bias"], a["qn"], a["kn"])
    txt = ((buf.fd, offs["act"] + image * k * 4), a["wt"], (-1, 0), a["qn"], a["kn"])
    p = h.qkv_dual_rope_params(a["q"], a["k"], a["v"], img, txt, a["pe"], image, text, k, n_heads, hd, 3, 70)
    rc, _ = h.execute(12, p)
    assert rc == 0, h.last_error()
    got = [buf.read(np.uint16, qkv_bytes // 2, offs[n]) for n in ("q", "k", "v")]
    raws = []
    for rows, wp in ((act[:image], pieces[1][1]), (act[image:], pieces[2][1])):
        raws.append(library_raw(dict(tokens=rows.shape[0], k=k, n_heads=n_heads, hd=hd, permuted=wp, act=rows)))
    ref = orc.qkv_post(raws[0], bias, qn, kn, pe, 3, tokens, image, n_heads, hd, tiles)
    ref = orc.qkv_post(raws[1], None, qn, kn, pe, 70, tokens, text, n_heads, hd, tiles, out_offset=image, out=ref)
    for which in range(3):
        assert np.array_equal(got[which], ref[which]), which


@pytest.mark.gpu
@pytest.mark.parametrize("tokens,n_heads,hd,rope,bias,offset,count,out_tile", [
    (1100, 24, 64, True, True, 0, 1100, 0),   # ragged last row tile (1100 = 8 * 128 + 76)
    (520, 24, 128, True, False, 7, 300, 1),   # rotary window, no bias, later output tiles
    (300, 30, 64, False, True, 0, 0, 0),
    (160, 38, 64, True, True, 0, 160, 2),
])
def test_hb_qkv_gemm_bit_exact(hip, orc, tokens, n_heads, hd, rope, bias, offset, count, out_tile):
    """The GEMM with the post-processing in its epilogue equals the oracle's
    post-processing of the library's GEMM output (hb_f16_gemm_ws)."""
    k = 256
    rng = np.random.default_rng(tokens + n_heads)
    cols = 3 * n_heads * hd
    act = rng.normal(0, 1, (tokens, k)).astype(np.float32)
    w = rng.normal(0, 0.05, (k, cols)).astype(np.float16)
    perm = h.permute_f16(w.view(np.uint16))
    _, b, qn, kn, pe = post_inputs(tokens, n_heads, hd, tokens, rope_tokens=offset + tokens + 3 if rope else 0)
    b = b if bias else None
    raw = library_raw(dict(tokens=tokens, k=k, n_heads=n_heads, hd=hd, permuted=perm, act=act))
    tiles = out_tile + (tokens + 31) // 32
    size = n_heads * orc.qkv_head_elems(tiles, hd)
    ref = orc.qkv_post(raw, b, qn, kn, pe, offset, count, tokens, n_heads, hd, tiles, out_offset=32 * out_tile,
                       out=tuple(np.full(size, 0x1234, np.uint16) for _ in range(3)))
    outs = [dev(np.full(size, 0x1234, np.uint16)) for _ in range(3)]
    packed = h.f16_prepack(dev(perm), k, cols)
    ws = h.DeviceBuffer(h.qkv_gemm_workspace_bytes(tokens, k))
    h.qkv_gemm(*outs, dev(act), packed, dev(b) if bias else None, dev(qn), dev(kn), dev(pe) if rope else None, offset,
               count, tokens, k, n_heads, hd, tiles, 32 * out_tile, ws)
    h.sync()
    for which, (o, r) in enumerate(zip(outs, ref)):
        got = o.read(np.uint16, size)
        assert np.array_equal(got, r), (which, int((got != r).sum()))


@pytest.mark.gpu
def test_hb_qkv_gemm_rejects_bad_arguments(hip):
    x = h.DeviceBuffer(1 << 20)
    ws = h.DeviceBuffer(1 << 20)
    args = (x, x, x, x, x, None, x, x, None, 0, 0)
    with pytest.raises(h.HtpOpsError):
        h.qkv_gemm(*args, 64, 256, 1, 64, 2, 0, ws)        # heads * head_dim not a multiple of 128
    with pytest.raises(h.HtpOpsError):
        h.qkv_gemm(*args, 64, 250, 2, 64, 2, 0, ws)        # input_dim not a multiple of 32
    with pytest.raises(h.HtpOpsError):
        h.qkv_gemm(*args, 4096, 4096, 2, 64, 128, 0, ws)   # workspace too small
    with pytest.raises(h.HtpOpsError):
        h.qkv_gemm(*args, 64, 256, 2, 64, 2, 32, ws)       # tokens past the output tiles
