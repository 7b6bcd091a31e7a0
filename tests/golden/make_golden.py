"""Writes the committed golden fixtures of this directory from the C oracle.

    python tests/golden/make_golden.py        (after `make -C oracle`)

The reference ships no golden vectors for opcodes 15/16 (its tests assert
only the integer HMX arithmetic), so these fixtures freeze the oracle's
outputs on small seeded inputs; tests/test_golden.py re-derives each one from
closed forms that do not go through the oracle (int64 brute force over the
decoded blob, per-op float32 numpy restatements, float64 F16 products) before
the GPU path is compared with them.

Files (numpy .npz, no pickled objects; load with allow_pickle=False):
  w8a8_golden.npz  per case <name>/: m,k,n (int64 scalars), x f32[m,k],
                   blob u8 (constants blob, reference op_reg.h:80-85 layout),
                   u u8[m,k], s f32[m], acc i32[m,n], y f32[m,n]
  f16_golden.npz   per case <name>/: m,k,n,channels,mode (int64 scalars),
                   x f32[m,k], w u16 (permuted fp16 weight, reference
                   test.c:547-558 layout), bias f32[channels] or absent, y f32
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as orc  # noqa: E402

# name: (m, k, n, seed, inv kind, sums kind, outlier fraction)
W8A8_CASES = {
    "c1_slice": (5, 64, 128, 0, "ones", "exact", 0.0),
    "tails": (17, 96, 192, 1, "uniform", "random", 0.05),
    "decode_row": (1, 160, 64, 2, "uniform", "exact", 0.0),
    "special_rows": (4, 32, 64, 3, "ones", "exact", 0.0),
}

# name: (m, k, n, channels, mode, with bias, seed)
F16_CASES = {
    "bias": (7, 64, 96, 96, 0, True, 10),
    "no_bias": (3, 32, 64, 64, 0, False, 11),
    "gelu": (7, 64, 96, 96, 1, True, 12),
    "quick_gelu": (9, 96, 64, 64, 2, True, 13),
    "channel_major": (5, 64, 96, 40, 3, True, 14),
}


def w8a8_case(m, k, n, seed, inv_kind, sums_kind, outliers):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    if outliers:
        chans = np.random.default_rng(seed + 7).choice(k, max(1, int(outliers * k)), replace=False)
        x[:, chans] *= 20.0
    if inv_kind == "ones":
        inv = np.ones(k, np.float32)
    else:
        inv = orc.uniform(k, 0.5, 2.0, seed + 3)
    if m == 4 and k == 32:
        # zero row (s = 1e-12, u = 128); a row whose max |t| is exactly 127
        # (s = 1, u = rne(t + 128): ties 0.5 -> 128, 1.5 -> 130, 2.5 -> 130,
        # -0.5 -> 128); a row of tiny values; a row with one huge value
        x[0] = 0.0
        x[1] = np.linspace(-3.5, 3.5, k, dtype=np.float32)
        x[1, :4] = [0.5, 1.5, 2.5, -0.5]
        x[1, 4] = 127.0
        x[2] = np.float32(1e-30) * np.arange(1, k + 1, dtype=np.float32)
        x[3, 7] = 3.0e4
    w = orc.int8_uniform(n * k, -127, 127, seed + 1).reshape(n, k)
    sw = orc.uniform(n, 1e-4, 1e-3, seed + 2)
    sums = None
    if sums_kind == "random":
        sums = np.random.default_rng(seed + 4).integers(-2**20, 2**20, n).astype(np.int32)
    blob = orc.pack_blob(w, sw, sums=sums, inv=inv, signature=seed)
    u, s = orc.quantize(x, inv)
    acc = orc.accumulate(u, blob, k, n)
    y = orc.linear(x, blob, k, n)
    return {"m": np.int64(m), "k": np.int64(k), "n": np.int64(n), "x": x, "blob": blob, "u": u, "s": s, "acc": acc,
            "y": y}


def f16_case(m, k, n, channels, mode, with_bias, seed):
    x = orc.normal(m * k, 0.0, 1.0, seed).reshape(m, k)
    w = orc.f32_to_f16_bits(orc.normal(k * n, 0.0, 0.05, seed + 1)).reshape(k, n)
    permuted = orc.f16_permute(w)
    bias = orc.normal(channels, 0.0, 0.02, seed + 2) if with_bias else None
    y = orc.f16_gemm_epilogue(x, permuted, bias, m, k, n, channels, mode)
    out = {"m": np.int64(m), "k": np.int64(k), "n": np.int64(n), "channels": np.int64(channels),
           "mode": np.int64(mode), "x": x, "w": permuted, "y": y}
    if bias is not None:
        out["bias"] = bias
    return out


def flatten(cases):
    flat = {}
    for name, arrays in cases.items():
        for key, value in arrays.items():
            flat[f"{name}/{key}"] = value
    return flat


def main():
    w8a8 = {name: w8a8_case(*args) for name, args in W8A8_CASES.items()}
    f16 = {name: f16_case(*args) for name, args in F16_CASES.items()}
    np.savez_compressed(os.path.join(HERE, "w8a8_golden.npz"), **flatten(w8a8))
    np.savez_compressed(os.path.join(HERE, "f16_golden.npz"), **flatten(f16))


if __name__ == "__main__":
    main()
