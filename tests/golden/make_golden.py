"""Writes the golden matmul fixtures under tests/golden/ (numpy float64).

Each fixture holds seeded float32 (or bf16-representable) operands stored as
flat buffers plus the view (shape, strides, offset) the matmul reads them
through, and the expected product computed in float64 by numpy's matmul on
the logical (already strided) operands.  These pin the oracle's view
handling, batch broadcasting and bf16 widening against an independent
library routine.  Run from the repo root: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
from scipy.special import erf

OUT = Path(__file__).resolve().parent


def bf16_round(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def view(buf, shape, strides, offset):
    es = buf.itemsize
    return np.lib.stride_tricks.as_strided(buf[offset:], shape=shape, strides=[s * es for s in strides])


def save(name, abuf, ash, ast, aoff, bbuf, bsh, bst, boff, dtype, extra=None):
    if dtype == "bf16":
        av = bf16_f32(view(abuf, ash, ast, aoff)).astype(np.float64)
        bv = bf16_f32(view(bbuf, bsh, bst, boff)).astype(np.float64)
    else:
        av = view(abuf, ash, ast, aoff).astype(np.float64)
        bv = view(bbuf, bsh, bst, boff).astype(np.float64)
    c = np.matmul(av, bv)
    absprod = np.matmul(np.abs(av), np.abs(bv))  # sum_k |a||b|, for the error bound
    d = dict(a_buf=abuf, a_shape=ash, a_strides=ast, a_offset=aoff, b_buf=bbuf, b_shape=bsh, b_strides=bst,
             b_offset=boff, dtype=dtype, expected=c, absprod=absprod)
    if extra:
        d.update(extra(c))
    np.savez_compressed(OUT / f"{name}.npz", **d)


def main():
    rng = np.random.default_rng(20260427)
    u = lambda n: rng.uniform(-1, 1, n).astype(np.float32)
    # 1. contiguous rectangular, f32
    M, K, N = 37, 53, 29
    save("f32_contiguous", u(M * K), [M, K], [K, 1], 0, u(K * N), [K, N], [N, 1], 0, "f32")
    # 2. B as a transposed view of an [N, K] buffer (strides [1, K])
    M, K, N = 40, 64, 24
    save("f32_b_transposed", u(M * K), [M, K], [K, 1], 0, u(N * K), [K, N], [1, K], 0, "f32")
    # 3. A as every other row of a bigger buffer, offset 3; A transposed as well in the B slot
    M, K, N = 21, 18, 26
    save("f32_a_strided_offset", u(3 + 2 * M * K), [M, K], [2 * K, 1], 3, u(K * N), [K, N], [N, 1], 0, "f32")
    # 4. flipped (negative-stride) A rows and transposed A
    M, K, N = 16, 20, 12
    save("f32_negative_stride", u(M * K), [M, K], [-K, 1], (M - 1) * K, u(N * K), [K, N], [1, K], 0, "f32")
    # 5. batched with broadcasting: A [3, 2, 9, 14] (every other row), B [2, 14, 11] -> [3, 2, 9, 11]
    ash = [3, 2, 9, 14]
    ast = [2 * 18 * 14, 18 * 14, 2 * 14, 1]
    save("f32_batched_broadcast", u(3 * 2 * 18 * 14), ash, ast, 0, u(2 * 14 * 11), [2, 14, 11], [154, 11, 1], 0,
         "f32")
    # 6. batch dim of extent 1 broadcast against 4 (the config-4 pattern)
    save("f32_batch1_broadcast", u(4 * 6 * 10), [4, 6, 10], [60, 10, 1], 0, u(10 * 7), [1, 10, 7], [70, 7, 1], 0,
         "f32")
    # 7. bf16 inputs, f32 accumulate: B a transposed view (the config-3 layout)
    M, K, N = 33, 96, 40
    abits = bf16_round(rng.normal(0, 1, M * K).astype(np.float32))
    bbits = bf16_round(rng.normal(0, 1, N * K).astype(np.float32))
    save("bf16_nt", abits, [M, K], [K, 1], 0, bbits, [K, N], [1, K], 0, "bf16")
    # 8. f32 with bias + GELU epilogue (expected in float64 with scipy's erf)
    M, K, N = 12, 24, 20
    bias = u(N)

    def gelu_extra(c):
        z = c + bias.astype(np.float64)
        return dict(bias=bias, preact=z, gelu=0.5 * z * (1 + erf(z / np.sqrt(2.0))))
    save("f32_bias_gelu", u(M * K), [M, K], [K, 1], 0, u(K * N), [K, N], [N, 1], 0, "f32", gelu_extra)


if __name__ == "__main__":
    main()
