"""Reverse-mode autograd: a tape over the HIP backend's ops.

The reference reserves ``oxmera-autograd`` (crates/oxmera-autograd/src/lib.rs:1-12)
and ``oxmera-nn`` (crates/oxmera-nn/src/lib.rs:1-12) but defines nothing yet.
This tape records every op on ``Var``s and sweeps them in reverse
topological order; every gradient is computed on the device by the same
backend ops (GEMMs for matmul, the elementwise / reduction kernels for the
rest).  Supported: matmul (batched, broadcast), add / sub / mul / div
(broadcasting; gradients summed back over broadcast dims), neg, exp, ln,
abs, sum, max (ties share the gradient equally), and the two fused nodes
of the Linear MLP:

  linear    h = act(x.W + b)       one GEMM, bias (+ GELU) fused; with GELU the same
                                   epilogue saves GELU'(z) of the pre-activation z
  mse_loss  mean((y - t)^2)        loss and dy in one pass

whose backward emits exactly the MLP's GEMMs:

  dW = x^T . dz          A is a transposed VIEW of x (no copy), f32 result
  dx = dz . W^T          B is a transposed VIEW of W; when x is the output of a
                         GELU layer and that layer's only consumer, the
                         product with the saved GELU'(z) is fused into this
                         GEMM (x.grad then holds dz, the gradient w.r.t. that
                         layer's pre-activation)
  db = sums over rows of dz, formed by whichever kernel produces dz (the MSE
                         pass, or the dx GEMM's epilogue) when that kernel's
                         output is dz's only contribution; otherwise one
                         column-sum pass

Gradients of a Var are accumulated over its consumers (in f32 when their
dtypes differ); a leaf's ``grad`` also accumulates over backward calls
until it is cleared.  Matmul gradients are f32 (GEMM accumulation);
elementwise gradients keep the dtype of the incoming gradient.
"""
from __future__ import annotations

from typing import Optional, Sequence

from . import _lib
from .backend import backend_for
from .core import DType, NotImplementedOp, ShapeMismatch
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

    @property
    def dtype(self):
        return self.t.dtype

    def backward(self) -> None:
        backward(self)

    # operator sugar over the functions below
    def __add__(self, o): return add(self, o)

    def __sub__(self, o): return sub(self, o)

    def __mul__(self, o): return mul(self, o)

    def __truediv__(self, o): return div(self, o)

    def __neg__(self): return neg(self)

    def __matmul__(self, o): return matmul(self, o)

    def exp(self): return exp(self)

    def ln(self): return ln(self)

    def abs(self): return abs_(self)

    def sum(self, axes: Sequence[int] = ()): return sum_(self, axes)

    def max(self, axes: Sequence[int] = ()): return max_(self, axes)


# ---- the sweep --------------------------------------------------------------------


class _Ctx:
    """State of one backward sweep: accumulated gradients per Var, how many
    recorded consumers each Var has, and which fused producer-side bias
    gradients are complete."""

    def __init__(self, be, consumers: dict):
        self.be = be
        self.consumers = consumers
        self.grads: dict = {}           # id(var) -> Tensor
        self.preact: dict = {}          # id(var) -> grad is w.r.t. the producer's pre-activation
        self.db_valid: set = set()      # id(_LinearNode) whose .db holds the complete bias gradient
        self.unit_seed: Optional[int] = None

    def single_consumer(self, v: "Var") -> bool:
        return self.consumers.get(id(v), 0) == 1

    def accumulate(self, v: "Var", g: Tensor, preact: bool = False) -> None:
        if not v.requires_grad:
            return
        k = id(v)
        if k not in self.grads:
            self.grads[k] = g
            self.preact[k] = preact
            return
        if preact or self.preact[k]:
            raise NotImplementedOp("a pre-activation gradient cannot be accumulated with another gradient")
        self.grads[k] = _add_grads(self.be, self.grads[k], g)


def _add_grads(be, a: Tensor, b: Tensor) -> Tensor:
    if a.dtype != b.dtype:
        a, b = be.convert(a, DType.F32), be.convert(b, DType.F32)
    return be.add(a, b)


def backward(root: Var) -> None:
    """Reverse-mode sweep from a one-element root (seed gradient 1)."""
    if root.node is None:
        raise NotImplementedOp("backward from a Var that no recorded op produced")
    n = 1
    for d in root.t.shape:
        n *= d
    if n != 1:
        raise ShapeMismatch(f"shape mismatch: backward needs a one-element root, got {list(root.t.shape)}")
    order, seen, consumers = [], set(), {}

    def visit(v: Var):
        if v.node is None or id(v.node) in seen:
            return
        seen.add(id(v.node))
        for p in v.node.parents():
            consumers[id(p)] = consumers.get(id(p), 0) + 1
            visit(p)
        order.append(v)

    visit(root)
    be = backend_for(root.t.device)
    ctx = _Ctx(be, consumers)
    seed = _unit(root.t.device, root.t.dtype).reshape(root.t.shape)
    ctx.unit_seed = id(seed)
    ctx.accumulate(root, seed)
    for v in reversed(order):
        g = ctx.grads.get(id(v))
        if g is None:
            continue
        v.node.backward(ctx, g, ctx.preact[id(v)])
    # publish: intermediates take this sweep's gradient, leaves accumulate
    ids = {id(v): v for v in order}
    for v in order:
        for p in v.node.parents():
            ids.setdefault(id(p), p)
    for k, v in ids.items():
        g = ctx.grads.get(k)
        if g is None or v is root:
            continue
        if v.node is None and v.grad is not None:
            v.grad = _add_grads(be, v.grad, g)
        else:
            v.grad = g
            v._grad_preact = ctx.preact[k]


# ---- helpers -----------------------------------------------------------------------

_UNITS: dict = {}


def _unit(device, dtype: DType) -> Tensor:
    """A one-element tensor holding 1 on ``device`` (the seed gradient, in the
    root's dtype), made once per device and dtype: a host copy per backward
    would synchronise the stream.  Gradients are never written in place, so
    sharing it is safe."""
    t = _UNITS.get((device, dtype))
    if t is None:
        import numpy as np
        t = _UNITS[(device, dtype)] = Tensor.from_numpy(np.ones((1,), np.float32), device, dtype)
    return t


def _as(be, t: Tensor, dtype: DType) -> Tensor:
    return be.convert(t, dtype) if t.dtype != dtype else t


def _unbroadcast(be, g: Tensor, shape: tuple) -> Tensor:
    """Sum g (of a broadcast result's shape) back to ``shape``."""
    shape = tuple(shape)
    if tuple(g.shape) == shape:
        return g
    lead = g.ndim - len(shape)
    axes = list(range(lead)) + [lead + d for d, e in enumerate(shape) if e == 1 and g.shape[lead + d] != 1]
    r = be.sum(g, axes) if axes else g
    return r.reshape(shape)


def _keepdims(t: Tensor, in_shape: tuple, axes: Sequence[int]) -> Tensor:
    """A reduction's result viewed with the reduced dims kept (extent 1)."""
    ax = set(axes) if len(axes) else set(range(len(in_shape)))
    return t.reshape(tuple(1 if d in ax else e for d, e in enumerate(in_shape)))


def _expand(be, t: Tensor, shape: tuple) -> Tensor:
    """t (extent-1 dims) repeated to ``shape``, materialised."""
    st = tuple(0 if (e == 1 and s != 1) else t.layout.strides[d] for d, (e, s) in enumerate(zip(t.shape, shape)))
    return be.contiguous(t.with_layout(shape, st, t.layout.offset))


def _rg(*vs) -> bool:
    return any(v is not None and v.requires_grad for v in vs)


def _var(x) -> Var:
    return x if isinstance(x, Var) else Var(x, False)


def _record(t: Tensor, node) -> Var:
    out = Var(t, node is not None, node)
    if node is not None:
        node.out = out
    return out


class _Node:
    out: Optional[Var] = None

    def parents(self):
        return [v for v in self.inputs if v is not None]


# ---- generic nodes -----------------------------------------------------------------


class _Binary(_Node):
    def __init__(self, op: int, a: Var, b: Var):
        self.op, self.inputs = op, (a, b)

    def backward(self, ctx, g: Tensor, preact: bool) -> None:
        be = ctx.be
        a, b = self.inputs
        dt = g.dtype
        A, B = _as(be, a.t, dt), _as(be, b.t, dt)
        if self.op == _lib.BIN_ADD:
            ga, gb = g, g
        elif self.op == _lib.BIN_SUB:
            ga, gb = g, (be.neg(g) if b.requires_grad else None)
        elif self.op == _lib.BIN_MUL:
            ga = be.mul(g, B) if a.requires_grad else None
            gb = be.mul(g, A) if b.requires_grad else None
        else:  # div: d(a/b)/da = 1/b, d(a/b)/db = -(a/b)/b
            ga = be.div(g, B) if a.requires_grad else None
            gb = be.neg(be.div(be.mul(g, _as(be, self.out.t, dt)), B)) if b.requires_grad else None
        if a.requires_grad:
            ctx.accumulate(a, _unbroadcast(be, ga, a.t.shape))
        if b.requires_grad:
            ctx.accumulate(b, _unbroadcast(be, gb, b.t.shape))


class _Unary(_Node):
    def __init__(self, op: int, a: Var):
        self.op, self.inputs = op, (a,)

    def backward(self, ctx, g: Tensor, preact: bool) -> None:
        be = ctx.be
        (a,) = self.inputs
        A = _as(be, a.t, g.dtype)
        if self.op == _lib.UN_NEG:
            ga = be.neg(g)
        elif self.op == _lib.UN_EXP:
            ga = be.mul(g, _as(be, self.out.t, g.dtype))
        elif self.op == _lib.UN_LN:
            ga = be.div(g, A)
        else:  # abs
            ga = be.mul(g, be.sign(A))
        ctx.accumulate(a, ga)


class _Sum(_Node):
    def __init__(self, a: Var, axes):
        self.inputs, self.axes = (a,), list(axes)

    def backward(self, ctx, g: Tensor, preact: bool) -> None:
        (a,) = self.inputs
        ctx.accumulate(a, _expand(ctx.be, _keepdims(g, a.t.shape, self.axes), a.t.shape))


class _Max(_Node):
    def __init__(self, a: Var, axes):
        self.inputs, self.axes = (a,), list(axes)

    def backward(self, ctx, g: Tensor, preact: bool) -> None:
        be = ctx.be
        (a,) = self.inputs
        A = _as(be, a.t, g.dtype)
        m = _keepdims(_as(be, self.out.t, g.dtype), a.t.shape, self.axes)
        mask = be.eq(A, m)
        cnt = _keepdims(be.sum(mask, self.axes), a.t.shape, self.axes)
        ctx.accumulate(a, be.mul(mask, be.div(_keepdims(g, a.t.shape, self.axes), cnt)))


class _Matmul(_Node):
    def __init__(self, a: Var, b: Var):
        self.inputs = (a, b)

    def backward(self, ctx, g: Tensor, preact: bool) -> None:
        be = ctx.be
        a, b = self.inputs
        if a.requires_grad:
            # dA = dC . B^T (B^T a stride view), summed over A's broadcast batch dims
            ga = be.matmul(_as(be, g, b.t.dtype), b.t.transpose_last(), out_dtype=DType.F32)
            ctx.accumulate(a, _unbroadcast(be, ga, a.t.shape))
        if b.requires_grad:
            gb = be.matmul(a.t.transpose_last(), _as(be, g, a.t.dtype), out_dtype=DType.F32)
            ctx.accumulate(b, _unbroadcast(be, gb, b.t.shape))


def _binary(op: int, a, b) -> Var:
    a, b = _var(a), _var(b)
    be = backend_for(a.t.device)
    t = be._binary(op, a.t, b.t)
    return _record(t, _Binary(op, a, b) if _rg(a, b) else None)


def _unary(op: int, a) -> Var:
    a = _var(a)
    t = backend_for(a.t.device)._unary(op, a.t)
    return _record(t, _Unary(op, a) if a.requires_grad else None)


def add(a, b) -> Var: return _binary(_lib.BIN_ADD, a, b)


def sub(a, b) -> Var: return _binary(_lib.BIN_SUB, a, b)


def mul(a, b) -> Var: return _binary(_lib.BIN_MUL, a, b)


def div(a, b) -> Var: return _binary(_lib.BIN_DIV, a, b)


def neg(a) -> Var: return _unary(_lib.UN_NEG, a)


def exp(a) -> Var: return _unary(_lib.UN_EXP, a)


def ln(a) -> Var: return _unary(_lib.UN_LN, a)


def abs_(a) -> Var: return _unary(_lib.UN_ABS, a)


def sum_(a, axes: Sequence[int] = ()) -> Var:
    a = _var(a)
    t = backend_for(a.t.device).sum(a.t, list(axes))
    return _record(t, _Sum(a, axes) if a.requires_grad else None)


def max_(a, axes: Sequence[int] = ()) -> Var:
    a = _var(a)
    t = backend_for(a.t.device).max(a.t, list(axes))
    return _record(t, _Max(a, axes) if a.requires_grad else None)


def matmul(a, b, out_dtype: DType | None = None) -> Var:
    """a . b (MatmulOps::matmul semantics: rank >= 2, batch dims broadcast);
    f32 result unless ``out_dtype`` is given."""
    a, b = _var(a), _var(b)
    t = backend_for(a.t.device).matmul(a.t, b.t, out_dtype=out_dtype)
    return _record(t, _Matmul(a, b) if _rg(a, b) else None)


# ---- the fused Linear / MSE nodes of the MLP -----------------------------------------


class _LinearNode(_Node):
    def __init__(self, x: Var, w: Var, b: Optional[Var], act: int, gd: Optional[Tensor]):
        # gd: GELU'(z) of the pre-activation z, saved by the forward epilogue
        self.x, self.w, self.b, self.act, self.gd = x, w, b, act, gd
        self.inputs = (x, w, b)
        self.db: Optional[Tensor] = None  # bias gradient formed by the producer of dz

    def wants_db(self) -> bool:
        return self.b is not None and self.b.requires_grad

    def backward(self, ctx, dout: Tensor, dout_is_preact: bool) -> None:
        be = ctx.be
        if self.act == _lib.ACT_GELU and not dout_is_preact:
            # the output fed something other than one Linear: dz = dout * GELU'(z)
            dz = be.mul(_as(be, dout, self.gd.dtype), self.gd)
        else:
            dz = dout  # gradient w.r.t. the pre-activation
        x2 = _rows(self.x.t)
        dz2 = _rows(dz)
        if self.w.requires_grad:
            # dW = x^T . dz  (x^T is a stride view)
            ctx.accumulate(self.w, be.matmul(x2.transpose_last(), _as(be, dz2, x2.dtype), out_dtype=DType.F32))
        if self.wants_db():
            db = self.db if (id(self) in ctx.db_valid and self.db is not None) else be.sum_rows_f32(dz2)
            ctx.accumulate(self.b, db)
        if self.x.requires_grad:
            prod = self.x.node
            fuse = isinstance(prod, _LinearNode) and prod.act == _lib.ACT_GELU and ctx.single_consumer(self.x)
            # dx = dz . W^T  (W^T is a stride view), GELU'(z_prev) fused when x = GELU(z_prev)
            # and this is x's only consumer; dx is then the producer's whole dz, and its
            # bias gradient comes out of the same epilogue
            db_prev = None
            if fuse and prod.wants_db():
                db_prev = Tensor.empty((self.w.t.shape[0],), DType.F32, dz.device)
            dx = be.matmul(_as(be, dz, self.w.t.dtype), self.w.t.transpose_last(), out_dtype=self.x.t.dtype,
                           act=_lib.ACT_MUL_AUX if fuse else _lib.ACT_NONE, aux=prod.gd if fuse else None,
                           colsum=db_prev)
            if db_prev is not None:
                prod.db = db_prev
                ctx.db_valid.add(id(prod))
            ctx.accumulate(self.x, dx, fuse)


def _rows(t: Tensor) -> Tensor:
    if t.ndim == 2:
        return t
    r = 1
    for d in t.shape[:-1]:
        r *= d
    return t.reshape((r, t.shape[-1]))


class _MSENode(_Node):
    def __init__(self, y: Var, dy: Tensor):
        self.y, self.dy = y, dy
        self.inputs = (y,)

    def backward(self, ctx, dout: Tensor, dout_is_preact: bool) -> None:
        # d(loss)/dy was produced with the loss, for a seed gradient of 1
        be = ctx.be
        prod = self.y.node
        if id(dout) == ctx.unit_seed:
            dy = self.dy
            if isinstance(prod, _LinearNode) and prod.db is not None and ctx.single_consumer(self.y):
                ctx.db_valid.add(id(prod))
        else:
            dy = be.mul(self.dy, _as(be, dout, self.dy.dtype))
        ctx.accumulate(self.y, dy)


def linear(x: Var, w: Var, b: Optional[Var] = None, act: int = _lib.ACT_NONE) -> Var:
    """y = act(x . w + b) with w stored [in, out] (as "XW" implies)."""
    be = backend_for(x.t.device)
    rg = _rg(x, w, b)
    # a GELU layer on the tape saves GELU'(z) from the same epilogue
    keep = act == _lib.ACT_GELU and rg
    out_shape = x.t.shape[:-1] + (w.t.shape[-1],)
    gd = Tensor.empty(out_shape, x.t.dtype, x.t.device) if keep else None
    y = be.matmul(x.t, w.t, out_dtype=x.t.dtype, bias=b.t if b is not None else None,
                  act=_lib.ACT_GELU_GRAD if keep else act, aux=gd)
    return _record(y, _LinearNode(x, w, b, act, gd) if rg else None)


def mse_loss(y: Var, target: Tensor) -> Var:
    """mean((y - t)^2) as a one-element F32 tensor; the gradient is formed in
    the same pass (and, when y comes from a Linear with a bias, that bias's
    gradient too)."""
    be = backend_for(y.t.device)
    prod = y.node
    db = None
    if y.requires_grad and isinstance(prod, _LinearNode) and prod.act == _lib.ACT_NONE and prod.wants_db():
        db = Tensor.empty((y.t.shape[-1],), DType.F32, y.t.device)
    loss, dy = be.mse_loss_grad(y.t, target, dy_colsum=db)
    if db is not None:
        prod.db = db
    return _record(loss, _MSENode(y, dy) if y.requires_grad else None)
