"""A minimal reverse-mode tape for Linear(+bias)(+GELU) layers and MSE.

The reference reserves ``oxmera-autograd`` (crates/oxmera-autograd/src/lib.rs:1-12)
and ``oxmera-nn`` (crates/oxmera-nn/src/lib.rs:1-12) but defines nothing yet;
this tape is what a Linear -> GELU -> Linear -> MSE model needs and emits
exactly the GEMMs of that model on the HIP backend:

  forward   h = GELU(x.W + b)      one GEMM, bias + GELU fused, pre-activation z kept
            y = h.W2 + b2          one GEMM, bias fused
  backward  dW = x^T . dz          A is a transposed VIEW of x (no copy)
            dx = dz . W^T          B is a transposed VIEW of W; when x came out of
                                   a GELU layer, GELU'(z) is fused into this GEMM
            db = sum over rows of dz, formed by whichever kernel produces dz:
                                   the MSE pass (dy) or the dx GEMM's epilogue
                                   (GELU' fused), from the values as stored

Weight and bias gradients are f32; activation gradients keep the
activation dtype.
"""
from __future__ import annotations

from typing import Optional

from . import _lib
from .backend import backend_for
from .core import DType, NotImplementedOp
from .tensor import Tensor


class Var:
    """A tensor on the tape."""

    def __init__(self, t: Tensor, requires_grad: bool = False, node=None):
        self.t = t
        self.requires_grad = requires_grad
        self.node = node
        self.grad: Optional[Tensor] = None

    @property
    def shape(self):
        return self.t.shape

    def backward(self) -> None:
        backward(self)


class _LinearNode:
    def __init__(self, x: Var, w: Var, b: Optional[Var], act: int, z: Optional[Tensor]):
        self.x, self.w, self.b, self.act, self.z = x, w, b, act, z
        self.out: Optional[Var] = None
        self.db: Optional[Tensor] = None  # bias gradient formed by the producer of dz

    def wants_db(self) -> bool:
        return self.b is not None and self.b.requires_grad

    def parents(self):
        return [v for v in (self.x, self.w, self.b) if v is not None]

    def backward(self, dout: Tensor, dout_is_preact: bool) -> None:
        be = backend_for(dout.device)
        if self.act == _lib.ACT_GELU and not dout_is_preact:
            raise NotImplementedOp("GELU backward without a fused producer GEMM")
        dz = dout  # gradient w.r.t. the pre-activation
        x2 = self.x.t.reshape((-1, self.x.t.shape[-1])) if self.x.t.ndim != 2 else self.x.t
        dz2 = dz.reshape((-1, dz.shape[-1])) if dz.ndim != 2 else dz
        if self.w.requires_grad:
            # dW = x^T . dz  (x^T is a stride view)
            _set_grad(self.w, be.matmul(x2.transpose_last(), dz2, out_dtype=DType.F32), False)
        if self.wants_db():
            _set_grad(self.b, self.db if self.db is not None else be.sum_rows_f32(dz2), False)
        if self.x.requires_grad:
            prod = self.x.node
            fuse = isinstance(prod, _LinearNode) and prod.act == _lib.ACT_GELU
            # dx = dz . W^T  (W^T is a stride view), GELU'(z_prev) fused when x = GELU(z_prev);
            # then dx is the producer layer's dz, and its bias gradient comes out of
            # the same epilogue
            db_prev = None
            if fuse and prod.wants_db():
                db_prev = Tensor.empty((self.w.t.shape[0],), DType.F32, dz.device)
            dx = be.matmul(dz, self.w.t.transpose_last(), out_dtype=self.x.t.dtype,
                           act=_lib.ACT_DGELU if fuse else _lib.ACT_NONE, aux=prod.z if fuse else None,
                           colsum=db_prev)
            if db_prev is not None:
                prod.db = db_prev
            _set_grad(self.x, dx, fuse)


class _MSENode:
    def __init__(self, y: Var, dy: Tensor):
        self.y, self.dy = y, dy

    def parents(self):
        return [self.y]

    def backward(self, dout: Tensor, dout_is_preact: bool) -> None:
        # d(loss)/dy was produced together with the loss (seed gradient 1).
        _set_grad(self.y, self.dy, False)


def _set_grad(v: Var, g: Tensor, preact: bool) -> None:
    if v.grad is not None:
        raise NotImplementedOp("gradient accumulation into a reused variable")
    v.grad = g
    v._grad_preact = preact


def linear(x: Var, w: Var, b: Optional[Var] = None, act: int = _lib.ACT_NONE) -> Var:
    """y = act(x . w + b) with w stored [in, out] (as "XW" implies)."""
    be = backend_for(x.t.device)
    keep_z = act == _lib.ACT_GELU and (x.requires_grad or w.requires_grad or (b is not None and b.requires_grad))
    out_shape = x.t.shape[:-1] + (w.t.shape[-1],)
    z = Tensor.empty(out_shape, x.t.dtype, x.t.device) if keep_z else None
    y = be.matmul(x.t, w.t, out_dtype=x.t.dtype, bias=b.t if b is not None else None, act=act, aux=z)
    rg = x.requires_grad or w.requires_grad or (b is not None and b.requires_grad)
    node = _LinearNode(x, w, b, act, z) if rg else None
    out = Var(y, rg, node)
    if node:
        node.out = out
    return out


def mse_loss(y: Var, target: Tensor) -> Var:
    """mean((y - t)^2) as a one-element F32 tensor; the gradient is formed in
    the same pass."""
    be = backend_for(y.t.device)
    prod = y.node
    db = None
    if y.requires_grad and isinstance(prod, _LinearNode) and prod.act == _lib.ACT_NONE and prod.wants_db():
        db = Tensor.empty((y.t.shape[-1],), DType.F32, y.t.device)  # its bias gradient, in the same pass
    loss, dy = be.mse_loss_grad(y.t, target, dy_colsum=db)
    if db is not None:
        prod.db = db
    node = _MSENode(y, dy) if y.requires_grad else None
    return Var(loss, y.requires_grad, node)


def backward(root: Var) -> None:
    """Reverse-mode sweep from a scalar root."""
    order, seen = [], set()

    def visit(v: Var):
        if v.node is None or id(v.node) in seen:
            return
        seen.add(id(v.node))
        for p in v.node.parents():
            visit(p)
        order.append(v)

    visit(root)
    for v in reversed(order):
        if v is root:
            v.node.backward(None, False)
        else:
            if v.grad is None:
                continue
            v.node.backward(v.grad, getattr(v, "_grad_preact", False))
