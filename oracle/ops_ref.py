"""CPU restatement of oxmera's UnaryOps / BinaryOps / ReduceOps and
Tensor::contiguous, the checker for the HIP backend's elementwise kernels.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and bench.py's checks), never
by the product package ``oxmera_amd``.

The reference defines only the contracts (crates/oxmera-ops/src/lib.rs:9-19,
27-69; crates/oxmera-tensor/src/tensor.rs:86-90); its CPU backend bodies are
``todo!()``.  Restated here with numpy, with the arithmetic points the
backend documents:
  * operands are read through their views (element strides, offsets);
  * binary ops broadcast per crates/oxmera-core/src/shape.rs:45-58 (NumPy);
  * 16-bit operands are widened exactly to f32, the op is one f32 operation
    (f64 for F64), and the result is rounded once (round to nearest even);
  * sum accumulates in f32 (f64 for F64) and rounds once; its order is not
    fixed by the contract, so checks of sums use the summation error bound;
  * max propagates NaN and has no identity for an empty extent.
Transcendentals (exp, ln) are computed here in float64 and rounded to the
dtype; the device's f32 functions may differ by a few f32 ulp, so checks
of exp/ln allow that.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

F32, F64, BF16, F16 = O.F32, O.F64, O.BF16, O.F16
UN_NEG, UN_EXP, UN_LN, UN_ABS = 0, 1, 2, 3
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = 0, 1, 2, 3


def to_f32(buf: np.ndarray, dtype: int) -> np.ndarray:
    """Exact widening of a raw buffer (bf16 bits, float16, float32, float64)."""
    if dtype == BF16:
        return O.bf16_to_f32(buf)
    if dtype == F16:
        return np.asarray(buf, np.float16).astype(np.float32)
    if dtype == F64:
        return np.asarray(buf, np.float64)
    return np.asarray(buf, np.float32)


def from_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    """Round once to the dtype's raw representation (RNE)."""
    if dtype == BF16:
        return O.bf16_round(np.asarray(x, np.float32))
    if dtype == F16:
        with np.errstate(over="ignore"):
            return np.asarray(x, np.float32).astype(np.float16)
    if dtype == F64:
        return np.asarray(x, np.float64)
    return np.asarray(x, np.float32)


def view(buf: np.ndarray, shape, strides, offset: int = 0) -> np.ndarray:
    """The logical array a strided view addresses (layout.rs:43-49)."""
    flat = buf.reshape(-1)
    es = flat.itemsize
    return np.lib.stride_tricks.as_strided(flat[offset:], shape=tuple(shape),
                                           strides=tuple(s * es for s in strides)).copy()


def broadcast_shape(a, b) -> tuple:
    """NumPy broadcasting (shape.rs:45-58); ValueError when incompatible."""
    out = []
    for i in range(1, max(len(a), len(b)) + 1):
        x = a[-i] if i <= len(a) else 1
        y = b[-i] if i <= len(b) else 1
        if x != y and x != 1 and y != 1:
            raise ValueError(f"shapes {list(a)} and {list(b)} do not broadcast")
        out.append(y if x == 1 else x)
    return tuple(reversed(out))


def unary(x: np.ndarray, op: int, dtype: int) -> np.ndarray:
    """UnaryOps (ops/src/lib.rs:27-37) on logical raw values x."""
    w = to_f32(x, dtype)
    acc = np.float64 if dtype == F64 else np.float32
    if op == UN_NEG:
        r = -w
    elif op == UN_ABS:
        r = np.abs(w)
    else:
        with np.errstate(divide="ignore", invalid="ignore"):
            r = (np.exp if op == UN_EXP else np.log)(w.astype(np.float64))
    return from_f32(np.asarray(r).astype(acc), dtype)


def binary(a: np.ndarray, b: np.ndarray, op: int, dtype: int) -> np.ndarray:
    """BinaryOps (ops/src/lib.rs:39-50): one f32 (f64) op per element after
    broadcasting, rounded once."""
    shape = broadcast_shape(a.shape, b.shape)
    x = np.broadcast_to(to_f32(a, dtype), shape)
    y = np.broadcast_to(to_f32(b, dtype), shape)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        r = [x + y, x - y, x * y, x / y][op]
    return from_f32(r, dtype)


def reduce_sum_f64(x: np.ndarray, axes, dtype: int) -> tuple[np.ndarray, np.ndarray]:
    """(float64 sum, float64 sum of |x|) over axes (empty = all), removing them
    (ops/src/lib.rs:61-66): the exact value and the scale of its error bound."""
    w = to_f32(x, dtype).astype(np.float64)
    ax = tuple(axes) if len(axes) else tuple(range(w.ndim))
    return w.sum(axis=ax), np.abs(w).sum(axis=ax)


def reduce_max(x: np.ndarray, axes, dtype: int) -> np.ndarray:
    """ReduceOps::max (ops/src/lib.rs:67-68): NaN propagates; an empty extent
    raises (no identity to invent)."""
    w = to_f32(x, dtype)
    ax = tuple(axes) if len(axes) else tuple(range(w.ndim))
    if any(w.shape[a] == 0 for a in ax):
        raise ValueError("max over an empty extent")
    return from_f32(np.max(w, axis=ax), dtype)


def reduced_shape(shape, axes) -> tuple:
    if not len(axes):
        return ()
    return tuple(e for d, e in enumerate(shape) if d not in set(axes))
