"""The HIP backend and the runtime registry, mirrored for the host side.

Mirrors:
  - ``Backend`` (crates/oxmera-runtime/src/lib.rs:25-34): every op family plus
    ``device()`` and ``name()``;
  - ``MatmulOps::matmul`` (crates/oxmera-ops/src/lib.rs:52-59), the hot path,
    served by ``oxm_gemm`` on gfx950;
  - ``ReduceOps::sum`` (ops/src/lib.rs:61-69) for axis 0 of a rank-2 tensor
    (the bias gradient), served by ``oxm_sum_rows``;
  - ``backend_for`` / ``register_backend`` (runtime/src/lib.rs:36-53): an
    unregistered device is ``BackendUnavailable``, never a crash.
Op families this backend does not carry raise ``NotImplementedOp``
(``Error::NotImplemented``, core/src/error.rs:92-101), never ``todo!``.
"""
from __future__ import annotations

import ctypes as C
import threading
from typing import Sequence

from . import _lib
from .core import (BackendUnavailable, Device, DType, NotImplementedOp, check)
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
            if colsum is not None and (colsum.dtype != DType.F32 or colsum.shape != (oshape[-1],)):
                raise ValueError(f"colsum must be F32 [{oshape[-1]}], got {colsum.dtype.name} {list(colsum.shape)}")
            ep = _lib.OxmEpilogue(C.c_void_p(bias.data_ptr() if bias is not None else 0),
                                  int(bias.dtype) if bias is not None else 0, int(act),
                                  C.c_void_p(aux.data_ptr() if aux is not None else 0),
                                  C.c_void_p(colsum.data_ptr() if colsum is not None else 0))
        check(_lib.lib().oxm_gemm(C.byref(a), C.byref(b), C.byref(c), C.byref(ep) if ep is not None else None,
                                  self._s(stream)))
        return out

    # ---- ReduceOps ----
    def sum(self, a: Tensor, axes: Sequence[int], *, stream: int | None = None) -> Tensor:
        if a.ndim != 2 or list(axes) != [0]:
            raise NotImplementedOp(f"sum is not implemented for rank {a.ndim} over axes {list(axes)} "
                                   "(hip backend: rank-2, axis 0)")
        out = Tensor.empty((a.shape[1],), DType.F32, a.device)
        x, o = a.abi_view(), out.abi_view()
        check(_lib.lib().oxm_sum_rows(C.byref(x), C.byref(o), self._s(stream)))
        return out

    def max(self, a: Tensor, axes: Sequence[int]) -> Tensor:
        raise NotImplementedOp("max is not implemented for the hip backend")

    # ---- UnaryOps / BinaryOps (not carried by this backend) ----
    def _absent(self, op: str):
        raise NotImplementedOp(f"{op} is not implemented for the hip backend")

    def neg(self, a): self._absent("neg")

    def exp(self, a): self._absent("exp")

    def ln(self, a): self._absent("ln")

    def abs(self, a): self._absent("abs")

    def add(self, lhs, rhs): self._absent("add")

    def sub(self, lhs, rhs): self._absent("sub")

    def mul(self, lhs, rhs): self._absent("mul")

    def div(self, lhs, rhs): self._absent("div")

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
