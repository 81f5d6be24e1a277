"""CPU reference of the 2-layer MLP training step (test infrastructure only).

The reference reserves oxmera-autograd / oxmera-nn (crates/oxmera-autograd/
src/lib.rs:1-12, crates/oxmera-nn/src/lib.rs:1-12) without defining them;
BASELINE.json's configs[4] defines the model: Linear d->h + bias + GELU,
Linear h->d + bias, MSE against a target, W stored [in, out] ("XW").

`step_oracle` composes the oracle GEMM (oracle/oxm_oracle.c) with the same
rounding points as the GPU path:
  G1 = bf16(GELU'(X.W1 + b1))   H = bf16(GELU(X.W1 + b1))   (both of the f32 value)
  Y  = bf16(H.W2 + b2)          loss = mean((Y - T)^2)      dY = bf16(2 (Y - T) / n)
  dW2 = H^T.dY (f32)            db2 = sum_rows dY (f32)
  dZ1 = bf16((dY.W2^T) * G1)
  dW1 = X^T.dZ1 (f32)           db1 = sum_rows dZ1 (f32)    dX = bf16(dZ1.W1^T)
`step_float64` is the same model in float64 with exact erf (no rounding),
and `loss_float64` its forward, for finite-difference checks.
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import oracle as O


def _view(bits: np.ndarray) -> O.StridedView:
    return O.StridedView.contiguous(bits, O.BF16)


def _tview(bits: np.ndarray) -> O.StridedView:
    """Transposed view of a contiguous 2-D bf16 buffer."""
    return _view(bits).permute([1, 0])


def step_oracle(x, w1, b1, w2, b2, t, nthreads=None):
    """All arguments are bf16 bit arrays (uint16).  Returns a dict of the
    forward/backward results (bf16 results as bits, f32 as float32)."""
    kw = dict(nthreads=nthreads)
    h, g1 = O.matmul(_view(x), _view(w1), out_dtype=O.BF16, bias=b1, bias_dtype=O.BF16, act=O.ACT_GELU_GRAD,
                     want_aux=True, **kw)
    y = O.matmul(_view(h), _view(w2), out_dtype=O.BF16, bias=b2, bias_dtype=O.BF16, **kw)
    yf, tf = O.bf16_to_f32(y), O.bf16_to_f32(t)
    d = (yf - tf).astype(np.float32)
    n = d.size
    loss = np.float32(np.sum(d.astype(np.float64) ** 2) / n)
    dy = O.bf16_round(d * np.float32(2.0 / n))
    dw2 = O.matmul(_tview(h), _view(dy), out_dtype=O.F32, **kw)
    db2 = O.colsum(dy, O.BF16)
    dz1 = O.matmul(_view(dy), _tview(w2), out_dtype=O.BF16, act=O.ACT_MUL_AUX, aux=g1, **kw)
    dw1 = O.matmul(_tview(x), _view(dz1), out_dtype=O.F32, **kw)
    db1 = O.colsum(dz1, O.BF16)
    dx = O.matmul(_view(dz1), _tview(w1), out_dtype=O.BF16, **kw)
    return dict(g1=g1, h=h, y=y, loss=loss, dy=dy, dw2=dw2, db2=db2, dz1=dz1, dw1=dw1, db1=db1, dx=dx)


def _gelu64(z):
    return 0.5 * z * (1.0 + erf(z / np.sqrt(2.0)))


def _dgelu64(z):
    return 0.5 * (1.0 + erf(z / np.sqrt(2.0))) + z * np.exp(-0.5 * z * z) / np.sqrt(2.0 * np.pi)


def loss_float64(x, w1, b1, w2, b2, t):
    z = x @ w1 + b1
    y = _gelu64(z) @ w2 + b2
    return float(np.mean((y - t) ** 2))


def step_float64(x, w1, b1, w2, b2, t):
    """Analytic forward/backward in float64 (inputs float64 arrays)."""
    z = x @ w1 + b1
    h = _gelu64(z)
    y = h @ w2 + b2
    d = y - t
    loss = float(np.mean(d ** 2))
    dy = 2.0 * d / d.size
    dw2 = h.T @ dy
    db2 = dy.sum(0)
    dz = (dy @ w2.T) * _dgelu64(z)
    dw1 = x.T @ dz
    db1 = dz.sum(0)
    dx = dz @ w1.T
    return dict(z1=z, g1=_dgelu64(z), h=h, y=y, loss=loss, dy=dy, dw2=dw2, db2=db2, dz1=dz, dw1=dw1, db1=db1,
                dx=dx)
