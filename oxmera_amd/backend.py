"""The HIP backend and the runtime registry, mirrored for the host side.

Mirrors:
  - ``Backend`` (crates/oxmera-runtime/src/lib.rs:25-34): every op family plus
    ``device()`` and ``name()``;
  - ``MatmulOps::matmul`` (crates/oxmera-ops/src/lib.rs:52-59), the hot path,
    served by ``oxm_gemm`` on gfx950;
  - ``UnaryOps`` / ``BinaryOps`` (ops/src/lib.rs:27-50) by ``oxm_unary`` /
    ``oxm_binary`` (NumPy broadcasting), ``ReduceOps::sum`` / ``max``
    (ops/src/lib.rs:61-69) by ``oxm_reduce``, all for F32/F64/BF16/F16;
    other dtypes are ``UnsupportedDType`` (typed, never a panic);
  - ``Tensor::contiguous`` (tensor/src/tensor.rs:86-90) by ``oxm_copy_view``;
  - ``backend_for`` / ``register_backend`` (runtime/src/lib.rs:36-53): an
    unregistered device is ``BackendUnavailable``, never a crash.
"""
from __future__ import annotations

import ctypes as C
import threading
from typing import Sequence

from . import _lib
from .core import (BackendUnavailable, Device, DeviceMismatch, DType, DTypeMismatch, NotImplementedOp,
                   ShapeMismatch, check)
from .tensor import Tensor


class HipBackend:
    """MI355X (gfx950) backend for one HIP device.

    With no stream every op is synchronous (the result can be read at once,
    as MatmulOps::matmul returns a value).  `set_stream(handle)` makes every
    op asynchronous on that hipStream_t; device storage is then recycled in
    that stream's order.
    """

    def __init__(self, index: int = 0, stream: int | None = None):
        self._device = Device.rocm(index)
        self.stream = stream

    def set_stream(self, stream: int | None) -> None:
        self.stream = stream or None

    def _s(self, stream):
        s = stream if stream is not None else self.stream
        return C.c_void_p(s) if s else None

    def device(self) -> Device:
        return self._device

    def name(self) -> str:
        return _lib.lib().oxm_backend_name().decode()

    # ---- MatmulOps ----
    def matmul(self, lhs: Tensor, rhs: Tensor, *, out_dtype: DType | None = None, bias: Tensor | None = None,
               act: int = _lib.ACT_NONE, aux: Tensor | None = None, out: Tensor | None = None,
               colsum: Tensor | None = None, stream: int | None = None) -> Tensor:
        """``lhs . rhs`` into a fresh contiguous tensor (or ``out``), with an
        optional fused epilogue (bias, GELU / GELU-backward).  Operands are any
        strided views; nothing is copied.  ``colsum`` (F32 [N]) receives the
        sums over rows of the output as stored (a bias gradient)."""
        a, b = lhs.abi_view(), rhs.abi_view()
        nd = C.c_int32(0)
        shp = (C.c_int64 * _lib.MAX_DIMS)()
        check(_lib.lib().oxm_gemm_infer(C.byref(a), C.byref(b), C.byref(nd), shp))
        oshape = tuple(shp[i] for i in range(nd.value))
        if out is None:
            odt = out_dtype if out_dtype is not None else DType.F32
            out = Tensor.empty(oshape, odt, lhs.device)
        c = out.abi_view()
        ep = None
        if bias is not None or act != _lib.ACT_NONE or aux is not None or colsum is not None:
            # the epilogue's buffers reach the C-ABI as raw pointers: their
            # dtype, shape, layout and device are checked here
            n = oshape[-1]
            for name, t, dts, shape in (("bias", bias, (DType.F32, DType.BF16, DType.F16), (n,)),
                                        ("aux", aux, (out.dtype,), tuple(out.shape)),
                                        ("colsum", colsum, (DType.F32,), (n,))):
                if t is None:
                    continue
                if t.dtype not in dts:
                    raise DTypeMismatch(f"dtype mismatch: expected {dts[0].name}, got {t.dtype.name} in matmul "
                                        f"({name})")
                if tuple(t.shape) != shape:
                    raise ShapeMismatch(f"shape mismatch: expected {list(shape)}, got {list(t.shape)} in matmul "
                                        f"({name})")
                if not t.layout.is_contiguous():
                    raise NotImplementedOp(f"matmul is not implemented for a non-contiguous {name}")
                if t.device != lhs.device:
                    raise DeviceMismatch(f"device mismatch: {lhs.device} vs {t.device} in matmul ({name})")
            ep = _lib.OxmEpilogue(C.c_void_p(bias.data_ptr() if bias is not None else 0),
                                  int(bias.dtype) if bias is not None else 0, int(act),
                                  C.c_void_p(aux.data_ptr() if aux is not None else 0),
                                  C.c_void_p(colsum.data_ptr() if colsum is not None else 0))
        check(_lib.lib().oxm_gemm(C.byref(a), C.byref(b), C.byref(c), C.byref(ep) if ep is not None else None,
                                  self._s(stream)))
        return out

    # ---- ReduceOps ----
    def _reduce(self, op: int, a: Tensor, axes: Sequence[int], stream) -> Tensor:
        ax = (C.c_int32 * max(1, len(axes)))(*[int(x) for x in axes])
        v = a.abi_view()
        nd = C.c_int32(0)
        shp = (C.c_int64 * _lib.MAX_DIMS)()
        check(_lib.lib().oxm_reduce_infer(C.byref(v), ax, len(axes), C.byref(nd), shp))
        out = Tensor.empty(tuple(shp[i] for i in range(nd.value)), a.dtype, a.device)
        o = out.abi_view()
        check(_lib.lib().oxm_reduce(op, C.byref(v), ax, len(axes), C.byref(o), self._s(stream)))
        return out

    def sum(self, a: Tensor, axes: Sequence[int], *, stream: int | None = None) -> Tensor:
        """Sum over ``axes``, removing them; empty ``axes`` = all (a rank-0 result)."""
        return self._reduce(_lib.RED_SUM, a, axes, stream)

    def max(self, a: Tensor, axes: Sequence[int], *, stream: int | None = None) -> Tensor:
        """Maximum over ``axes``; an empty reduced extent is a typed error."""
        return self._reduce(_lib.RED_MAX, a, axes, stream)

    def sum_rows_f32(self, a: Tensor, *, stream: int | None = None) -> Tensor:
        """Column sums of a rank-2 tensor with an F32 result whatever a's dtype
        (the bias gradient of a Linear layer when no producer formed it)."""
        out = Tensor.empty((a.shape[1],), DType.F32, a.device)
        x, o = a.abi_view(), out.abi_view()
        check(_lib.lib().oxm_sum_rows(C.byref(x), C.byref(o), self._s(stream)))
        return out

    # ---- UnaryOps / BinaryOps ----
    def _unary(self, op: int, a: Tensor, stream=None) -> Tensor:
        out = Tensor.empty(a.shape, a.dtype, a.device)
        x, o = a.abi_view(), out.abi_view()
        check(_lib.lib().oxm_unary(op, C.byref(x), C.byref(o), self._s(stream)))
        return out

    def _binary(self, op: int, lhs: Tensor, rhs: Tensor, stream=None) -> Tensor:
        from .core import broadcast_shapes
        out = Tensor.empty(tuple(broadcast_shapes(lhs.shape, rhs.shape)), lhs.dtype, lhs.device)
        x, y, o = lhs.abi_view(), rhs.abi_view(), out.abi_view()
        check(_lib.lib().oxm_binary(op, C.byref(x), C.byref(y), C.byref(o), self._s(stream)))
        return out

    def neg(self, a, *, stream=None): return self._unary(_lib.UN_NEG, a, stream)

    def exp(self, a, *, stream=None): return self._unary(_lib.UN_EXP, a, stream)

    def ln(self, a, *, stream=None): return self._unary(_lib.UN_LN, a, stream)

    def abs(self, a, *, stream=None): return self._unary(_lib.UN_ABS, a, stream)

    def add(self, lhs, rhs, *, stream=None): return self._binary(_lib.BIN_ADD, lhs, rhs, stream)

    def sub(self, lhs, rhs, *, stream=None): return self._binary(_lib.BIN_SUB, lhs, rhs, stream)

    def mul(self, lhs, rhs, *, stream=None): return self._binary(_lib.BIN_MUL, lhs, rhs, stream)

    def div(self, lhs, rhs, *, stream=None): return self._binary(_lib.BIN_DIV, lhs, rhs, stream)

    # ---- what the autograd tape adds (no counterpart among the reference's ops) ----
    def sign(self, a, *, stream=None):
        """-1, 0 or +1 per element (NaN stays NaN): abs's derivative."""
        return self._unary(_lib.UN_SIGN, a, stream)

    def eq(self, lhs, rhs, *, stream=None):
        """1 where lhs == rhs else 0, broadcasting: max's gradient mask."""
        return self._binary(_lib.BIN_EQ, lhs, rhs, stream)

    def dgelu(self, grad, z, *, stream=None):
        """grad * GELU'(z) (erf GELU): the gradient through a GELU."""
        return self._binary(_lib.BIN_DGELU, grad, z, stream)

    def convert(self, a: Tensor, dtype: DType, *, stream: int | None = None) -> Tensor:
        """a in ``dtype`` (fresh contiguous storage), rounded once to nearest
        even; a itself when it already has that dtype."""
        if a.dtype == dtype:
            return a
        out = Tensor.empty(a.shape, dtype, a.device)
        x, o = a.abi_view(), out.abi_view()
        check(_lib.lib().oxm_convert(C.byref(x), C.byref(o), self._s(stream)))
        return out

    def sgd_step(self, param: Tensor, grad: Tensor, velocity: Tensor | None, lr: float, momentum: float = 0.0,
                 weight_decay: float = 0.0, nesterov: bool = False, *, stream: int | None = None) -> None:
        """One fused SGD update of ``param`` in place (oxm_sgd_step)."""
        p, g = param.abi_view(), grad.abi_view()
        v = velocity.abi_view() if velocity is not None else None
        check(_lib.lib().oxm_sgd_step(C.byref(p), C.byref(g), C.byref(v) if v is not None else None, float(lr),
                                      float(momentum), float(weight_decay), int(bool(nesterov)), self._s(stream)))

    # ---- Tensor::contiguous ----
    def contiguous(self, a: Tensor, *, stream: int | None = None) -> Tensor:
        """a's elements in logical order in fresh contiguous storage; a itself
        (sharing storage) when already contiguous (tensor.rs:86-90)."""
        if a.layout.is_contiguous():
            return a
        out = Tensor.empty(a.shape, a.dtype, a.device)
        x, o = a.abi_view(), out.abi_view()
        check(_lib.lib().oxm_copy_view(C.byref(x), C.byref(o), self._s(stream)))
        return out

    # ---- loss (MSE and its gradient in one pass) ----
    def mse_loss_grad(self, y: Tensor, t: Tensor, *, dy_colsum: Tensor | None = None,
                      stream: int | None = None) -> tuple[Tensor, Tensor]:
        """(loss, dy); ``dy_colsum`` (F32 [C]) also receives the sums of dy over
        its leading dimensions, in the same pass."""
        loss = Tensor.empty((1,), DType.F32, y.device)
        dy = Tensor.empty(y.shape, y.dtype, y.device)
        vy, vt, vl, vd = y.abi_view(), t.abi_view(), loss.abi_view(), dy.abi_view()
        vc = dy_colsum.abi_view() if dy_colsum is not None else None
        check(_lib.lib().oxm_mse_loss_grad(C.byref(vy), C.byref(vt), C.byref(vl), C.byref(vd),
                                           C.byref(vc) if vc is not None else None, self._s(stream)))
        return loss, dy


# ---- the registry (runtime/src/lib.rs:36-53) -----------------------------------

_REGISTRY: dict[Device, object] = {}
_LOCK = threading.Lock()


def register_backend(backend) -> None:
    """Register a backend for its device, replacing any previous one."""
    with _LOCK:
        _REGISTRY[backend.device()] = backend


def backend_for(device: Device):
    """The backend serving ``device``; BackendUnavailable when none is registered."""
    with _LOCK:
        b = _REGISTRY.get(device)
    if b is None:
        raise BackendUnavailable(f"no backend available for device {device!r}")
    return b


def device_count() -> int:
    n = C.c_int32(0)
    st = _lib.lib().oxm_device_count(C.byref(n))
    return n.value if st == _lib.OK else 0


def init() -> int:
    """Register a HipBackend for every visible HIP device; returns the count."""
    n = device_count()
    for i in range(n):
        register_backend(HipBackend(i))
    return n
