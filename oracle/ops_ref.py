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


# ---- integer and boolean dtypes ------------------------------------------------
# The reference's DType carries I32, I64, U8 and Bool (crates/oxmera-core/src/
# dtype.rs:9-22) but specifies no integer semantics beyond "integer division
# by zero is a typed error" (crates/oxmera-ops/src/lib.rs:47-48).  The build
# defines them as Rust's wrapping arithmetic on fixed-width integers (NumPy's
# fixed-width integer arithmetic is the same), `/` truncating toward zero,
# and Bool as a 0/1 byte with add = OR, mul = AND.  Restated with explicit
# integer operations here (no float round trips), so results are exact.

I32, I64, U8, BOOL = 2, 3, 4, 5
INT_NP = {I32: np.int32, I64: np.int64, U8: np.uint8, BOOL: np.uint8}
BIN_EQ = 4


class DivisionByZero(Exception):
    """Integer division by zero (the typed error of BinaryOps::div)."""


def _wrap(x: np.ndarray, dtype: int) -> np.ndarray:
    """Reduce an int64-or-object array modulo 2^bits into the dtype."""
    t = INT_NP[dtype]
    bits = np.iinfo(t).bits
    v = np.asarray(np.asarray(x, dtype=object) % (1 << bits), dtype=object)
    if np.iinfo(t).min < 0:
        v = np.asarray(np.where(v >= (1 << (bits - 1)), v - (1 << bits), v), dtype=object)
    return v.astype(t)


def int_unary(x: np.ndarray, op: int, dtype: int) -> np.ndarray:
    """neg / abs, wrapping; Bool: abs only (the identity)."""
    xo = np.asarray(x).astype(object)
    if dtype == BOOL:
        if op != UN_ABS:
            raise ValueError("Bool carries abs only")
        return np.asarray(x).copy()
    if op == UN_NEG:
        return _wrap(-xo, dtype)
    if op == UN_ABS:
        return _wrap(np.abs(xo), dtype)
    raise ValueError("integer dtypes carry neg and abs only")


def _trunc_div(a: int, b: int) -> int:
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def int_binary(a: np.ndarray, b: np.ndarray, op: int, dtype: int) -> np.ndarray:
    """add / sub / mul / div / eq with broadcasting; wrapping; div truncates
    toward zero and raises DivisionByZero for any zero divisor."""
    a, b = np.broadcast_arrays(np.asarray(a), np.asarray(b))
    if op == BIN_EQ:
        return (a == b).astype(INT_NP[dtype])
    if dtype == BOOL:
        if op == BIN_ADD:
            return ((a != 0) | (b != 0)).astype(np.uint8)
        if op == BIN_MUL:
            return ((a != 0) & (b != 0)).astype(np.uint8)
        raise ValueError("Bool carries add, mul and eq only")
    ao, bo = a.astype(object), b.astype(object)
    if op == BIN_ADD:
        return _wrap(ao + bo, dtype)
    if op == BIN_SUB:
        return _wrap(ao - bo, dtype)
    if op == BIN_MUL:
        return _wrap(ao * bo, dtype)
    if op == BIN_DIV:
        if np.any(b == 0):
            raise DivisionByZero("integer division by zero")
        q = np.frompyfunc(_trunc_div, 2, 1)(ao, bo)
        return _wrap(q, dtype)
    raise ValueError(op)


def int_reduce(x: np.ndarray, axes, op: int, dtype: int) -> np.ndarray:
    """sum (exact, then wrapped into the dtype) or max over `axes` (all when
    empty); Bool: both are OR.  max over an empty extent has no identity."""
    x = np.asarray(x)
    ax = tuple(range(x.ndim)) if len(axes) == 0 else tuple(axes)
    if dtype == BOOL:
        return np.any(x != 0, axis=ax).astype(np.uint8)
    if op == 0:  # sum
        return _wrap(np.sum(x.astype(object), axis=ax), dtype)
    if any(x.shape[a] == 0 for a in ax):
        raise ValueError("max over an empty extent")
    return np.max(x, axis=ax)
