"""CPU restatement of the gradients the autograd tape computes, and of the
SGD update, the checkers for ``oxmera_amd.autograd`` / ``oxmera_amd.optim``.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

The reference reserves oxmera-autograd, oxmera-nn and oxmera-optim
(crates/oxmera-autograd/src/lib.rs:1-12, crates/oxmera-nn/src/lib.rs:1-12,
crates/oxmera-optim/src/lib.rs:1-11) and defines nothing in them, so the
contract here is the calculus of the ops oxmera does define
(crates/oxmera-ops/src/lib.rs:27-69): vector-Jacobian products in float64
with NumPy broadcasting (crates/oxmera-core/src/shape.rs:45-58), pinned on
the CPU by central finite differences; SGD as torch.optim.SGD with
dampening 0, restated in float32 one rounded operation at a time, pinned by
closed forms.
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import oracle as O

ADD, SUB, MUL, DIV = 0, 1, 2, 3
NEG, EXP, LN, ABS = 0, 1, 2, 3


def unbroadcast(g: np.ndarray, shape) -> np.ndarray:
    """Sum g over the dims a broadcast added or stretched, back to ``shape``."""
    shape = tuple(shape)
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    for d, e in enumerate(shape):
        if e == 1 and g.shape[d] != 1:
            g = g.sum(axis=d, keepdims=True)
    return g


def binary(op: int, a, b):
    return {ADD: np.add, SUB: np.subtract, MUL: np.multiply, DIV: np.divide}[op](a, b)


def vjp_binary(op: int, a: np.ndarray, b: np.ndarray, g: np.ndarray):
    """(dL/da, dL/db) given g = dL/d(a op b)."""
    if op == ADD:
        ga, gb = g, g
    elif op == SUB:
        ga, gb = g, -g
    elif op == MUL:
        ga, gb = g * b, g * a
    else:
        ga, gb = g / b, -g * a / (b * b)
    return unbroadcast(np.broadcast_to(ga, g.shape), a.shape), unbroadcast(np.broadcast_to(gb, g.shape), b.shape)


def unary(op: int, a):
    return {NEG: np.negative, EXP: np.exp, LN: np.log, ABS: np.abs}[op](a)


def vjp_unary(op: int, a: np.ndarray, g: np.ndarray) -> np.ndarray:
    if op == NEG:
        return -g
    if op == EXP:
        return g * np.exp(a)
    if op == LN:
        return g / a
    return g * np.sign(a)


def _ax(a: np.ndarray, axes) -> tuple:
    return tuple(axes) if len(axes) else tuple(range(a.ndim))


def vjp_sum(a: np.ndarray, axes, g: np.ndarray) -> np.ndarray:
    return np.broadcast_to(np.expand_dims(g, _ax(a, axes)), a.shape).copy()


def vjp_max(a: np.ndarray, axes, g: np.ndarray) -> np.ndarray:
    """Ties share the gradient equally (the subgradient torch.amax uses)."""
    ax = _ax(a, axes)
    m = a.max(axis=ax, keepdims=True)
    mask = (a == m).astype(np.float64)
    return mask * np.expand_dims(g, ax) / mask.sum(axis=ax, keepdims=True)


def vjp_matmul(a: np.ndarray, b: np.ndarray, g: np.ndarray):
    """C = a @ b over broadcast batch dims (MatmulOps::matmul,
    crates/oxmera-ops/src/lib.rs:52-59): dA = g b^T, dB = a^T g, each summed
    over its operand's broadcast dims."""
    ga = g @ np.swapaxes(b, -1, -2)
    gb = np.swapaxes(a, -1, -2) @ g
    return unbroadcast(ga, a.shape), unbroadcast(gb, b.shape)


def gelu(z):
    return 0.5 * z * (1.0 + erf(z / np.sqrt(2.0)))


def dgelu(z):
    return 0.5 * (1.0 + erf(z / np.sqrt(2.0))) + z * np.exp(-0.5 * z * z) / np.sqrt(2.0 * np.pi)


def vjp_linear_gelu(x, w, b, g):
    """h = GELU(x w + b): (dx, dw, db) given g = dL/dh."""
    z = x @ w + b
    dz = g * dgelu(z)
    return dz @ w.T, x.T @ dz, dz.sum(axis=0)


# ---- SGD ---------------------------------------------------------------------------

def sgd_step(p_raw: np.ndarray, p_dtype: int, g: np.ndarray, v, lr, momentum=0.0, weight_decay=0.0,
             nesterov=False):
    """One step; returns (new raw param, new velocity or None).  p_raw: raw
    values of p_dtype (bf16 as uint16 bits); g: float32 values (the exact
    widening of the gradient); v: float32 or None.  Every operation is a
    float32 operation rounded on its own; p is rounded once at the end."""
    f = np.float32
    p = O.bf16_to_f32(p_raw) if p_dtype == O.BF16 else np.asarray(p_raw).astype(np.float32)
    g = np.asarray(g, np.float32)
    lr, mu, wd = f(lr), f(momentum), f(weight_decay)
    if wd != 0:
        g = g + wd * p
    if mu != 0:
        v = mu * np.asarray(v, np.float32) + g
        g = g + mu * v if nesterov else v
    new = p - lr * g
    if p_dtype == O.BF16:
        return O.bf16_round(new), v
    if p_dtype == O.F16:
        return new.astype(np.float16), v
    return new.astype(np.float32), v
