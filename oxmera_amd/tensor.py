"""Storage and Tensor views for the HIP backend's host side.

Mirrors ``crates/oxmera-tensor/src``:
  - ``Storage``: an owned, refcounted byte buffer on one device
    (storage.rs:12-68); device buffers come from ``oxm_alloc`` and are freed
    when the last view drops it ("GPU variants hold opaque backend handles",
    storage.rs:19-24).
  - ``Tensor``: a Layout over shared Storage (tensor.rs:15-19) with the view
    operations ``permute``/``narrow``/``reshape`` (tensor.rs:63-84), which never
    copy, and ``get_f32`` (tensor.rs:92-99).
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _lib
from .core import (Device, DType, IndexOutOfBounds, Layout, NotImplementedOp, OxmError, RankMismatch,
                   ShapeMismatch, check, contiguous_strides, numel)

# ---- host-side dtype conversion (data preparation, not compute) --------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest-even) and return the uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _np_dtype(dt: DType):
    return {DType.F32: np.float32, DType.F64: np.float64, DType.I32: np.int32, DType.I64: np.int64,
            DType.U8: np.uint8, DType.Bool: np.bool_, DType.BF16: np.uint16, DType.F16: np.float16}[dt]


def _copy_stream(device: Device):
    """The stream host copies of ``device`` run on: the registered backend's
    current stream, so that a copy is ordered after the kernels queued there
    (they may still read a recycled block, or produce the data being read);
    None (synchronous, device-wide) when no backend stream is set."""
    from .backend import _REGISTRY
    be = _REGISTRY.get(device)
    s = getattr(be, "stream", None) if be is not None else None
    return C.c_void_p(s) if s else None


# ---- storage -------------------------------------------------------------------


class _DevicePool:
    """Caching allocator for device storage (one per device).

    Freed blocks are kept per exact byte size and handed out again instead of
    calling hipFree (which synchronises the device).  Reuse is safe for work
    issued in stream order on one stream -- the backend's -- like PyTorch's
    caching allocator: every op and every host copy (``from_numpy``,
    ``to_numpy``) of a device runs on its backend's current stream, so a block
    handed out again is written only after the work that last used it.  Work
    issued on another stream must keep its tensors alive until that stream
    is synchronised.  `release()` returns everything to HIP.
    """

    def __init__(self, device: int, cap_bytes: int = 64 << 30):
        self.device = device
        self.cap = cap_bytes
        self.free: dict[int, list[int]] = {}
        self.cached = 0

    def get(self, nbytes: int) -> int:
        lst = self.free.get(nbytes)
        if lst:
            self.cached -= nbytes
            return lst.pop()
        p = C.c_void_p()
        st = _lib.lib().oxm_alloc(self.device, nbytes, C.byref(p))
        if st != _lib.OK:  # out of memory: give the cache back and retry once
            self.release()
            st = _lib.lib().oxm_alloc(self.device, nbytes, C.byref(p))
        check(st)
        return p.value

    def put(self, ptr: int, nbytes: int) -> None:
        if self.cached + nbytes > self.cap:
            _lib.lib().oxm_free(self.device, C.c_void_p(ptr))
            return
        self.free.setdefault(nbytes, []).append(ptr)
        self.cached += nbytes

    def release(self) -> None:
        for lst in self.free.values():
            for ptr in lst:
                _lib.lib().oxm_free(self.device, C.c_void_p(ptr))
        self.free.clear()
        self.cached = 0


_POOLS: dict[int, _DevicePool] = {}


def device_pool(index: int) -> _DevicePool:
    pool = _POOLS.get(index)
    if pool is None:
        pool = _POOLS[index] = _DevicePool(index)
    return pool


class Storage:
    """A byte buffer on one device; host storage wraps a numpy byte array,
    device storage is a block of the device's caching allocator."""

    def __init__(self, nbytes: int, dtype: DType, device: Device):
        self.nbytes = int(nbytes)
        self.dtype = DType(dtype)
        self.device = device
        self._host = None
        self._ptr = None
        if device.kind == "cpu":
            self._host = np.zeros(max(1, self.nbytes), dtype=np.uint8)
        else:
            self._ptr = device_pool(device.index).get(max(1, self.nbytes))

    @property
    def ptr(self) -> int:
        if self._host is not None:
            return self._host.ctypes.data
        return self._ptr

    def __del__(self):
        if getattr(self, "_ptr", None):
            try:
                device_pool(self.device.index).put(self._ptr, max(1, self.nbytes))
            except Exception:
                pass
            self._ptr = None


# ---- tensor -------------------------------------------------------------------


class Tensor:
    """A strided view over shared storage."""

    def __init__(self, storage: Storage, layout: Layout):
        self._storage = storage
        self._layout = layout

    # -- constructors --
    @staticmethod
    def from_storage(storage: Storage, layout: Layout) -> "Tensor":
        """A view with an explicit layout; errors when it addresses bytes
        outside the storage (tensor.rs:21-28)."""
        if numel(layout.shape) > 0:
            lo = hi = layout.offset
            for d, s in zip(layout.shape, layout.strides):
                span = (d - 1) * s
                lo, hi = (lo + span, hi) if span < 0 else (lo, hi + span)
            es = storage.dtype.size_in_bytes()
            if lo < 0 or (hi + 1) * es > storage.nbytes:
                raise IndexOutOfBounds(f"layout {layout} addresses elements outside a storage of "
                                       f"{storage.nbytes // es} elements", None, layout.shape)
        return Tensor(storage, layout)

    @staticmethod
    def empty(shape: Sequence[int], dtype: DType, device: Device) -> "Tensor":
        shape = tuple(int(d) for d in shape)
        st = Storage(numel(shape) * DType(dtype).size_in_bytes(), dtype, device)
        return Tensor(st, Layout.contiguous(shape))

    @staticmethod
    def from_numpy(arr: np.ndarray, device: Device, dtype: DType | None = None) -> "Tensor":
        """Copy a host array into fresh contiguous storage on ``device``.
        For BF16, float input is rounded to nearest-even; uint16 input is
        taken as raw bf16 bits."""
        arr = np.asarray(arr)
        if dtype is None:
            dtype = {np.dtype(np.float32): DType.F32, np.dtype(np.float64): DType.F64,
                     np.dtype(np.float16): DType.F16, np.dtype(np.int32): DType.I32,
                     np.dtype(np.int64): DType.I64, np.dtype(np.uint8): DType.U8,
                     np.dtype(np.bool_): DType.Bool}[arr.dtype]
        dtype = DType(dtype)
        if dtype == DType.BF16:
            host = arr if arr.dtype == np.uint16 else f32_to_bf16_bits(arr.astype(np.float32))
        else:
            host = arr.astype(_np_dtype(dtype))
        if not host.flags.c_contiguous:
            host = host.copy(order="C")  # (np.ascontiguousarray would turn a 0-d array into shape (1,))
        t = Tensor.empty(host.shape, dtype, device)
        t._storage_write(host)
        return t

    @staticmethod
    def from_vec_f32(data: Sequence[float], shape: Sequence[int], device: Device | None = None) -> "Tensor":
        """A contiguous F32 tensor (tensor.rs:30-36); errors when the length
        does not match the shape."""
        if len(data) != numel(shape):
            raise ShapeMismatch(f"shape mismatch: expected {[numel(shape)]}, got {[len(data)]} in from_vec_f32")
        return Tensor.from_numpy(np.asarray(data, dtype=np.float32).reshape(tuple(shape)),
                                 device or Device.cpu(), DType.F32)

    def _storage_write(self, host: np.ndarray) -> None:
        nbytes = host.nbytes
        if nbytes == 0:
            return
        if self.device.kind == "cpu":
            self._storage._host[:nbytes] = host.reshape(-1).view(np.uint8)
        else:
            check(_lib.lib().oxm_copy(C.c_void_p(self._storage.ptr), self.device.index,
                                      C.c_void_p(host.ctypes.data), -1, nbytes, _copy_stream(self.device)))

    # -- accessors --
    @property
    def shape(self) -> tuple[int, ...]:
        return self._layout.shape

    @property
    def layout(self) -> Layout:
        return self._layout

    @property
    def dtype(self) -> DType:
        return self._storage.dtype

    @property
    def device(self) -> Device:
        return self._storage.device

    @property
    def storage(self) -> Storage:
        return self._storage

    @property
    def ndim(self) -> int:
        return len(self._layout.shape)

    def data_ptr(self) -> int:
        """Address of element 0 of the view."""
        return self._storage.ptr + self._layout.offset * self.dtype.size_in_bytes()

    # -- views (never copy) --
    def permute(self, perm: Sequence[int]) -> "Tensor":
        n = self.ndim
        if len(perm) != n or sorted(perm) != list(range(n)):
            raise RankMismatch(f"permute: {list(perm)} is not a permutation of 0..{n}", len(perm), n)
        L = self._layout
        return Tensor(self._storage, Layout(tuple(L.shape[p] for p in perm), tuple(L.strides[p] for p in perm),
                                            L.offset))

    def transpose_last(self) -> "Tensor":
        """Swap the last two dims (a view)."""
        perm = list(range(self.ndim))
        perm[-1], perm[-2] = perm[-2], perm[-1]
        return self.permute(perm)

    def narrow(self, dim: int, start: int, length: int) -> "Tensor":
        L = self._layout
        if not 0 <= dim < self.ndim:
            raise RankMismatch(f"narrow: dim {dim} of a rank-{self.ndim} tensor", dim, self.ndim)
        if start < 0 or length < 0 or start + length > L.shape[dim]:
            raise IndexOutOfBounds(f"narrow: [{start}, {start + length}) outside extent {L.shape[dim]}",
                                   [start + length], L.shape)
        shape = list(L.shape)
        shape[dim] = length
        return Tensor(self._storage, Layout(tuple(shape), L.strides, L.offset + start * L.strides[dim]))

    def reshape(self, shape: Sequence[int]) -> "Tensor":
        shape = tuple(int(d) for d in shape)
        if numel(shape) != numel(self.shape):
            raise ShapeMismatch(f"shape mismatch: expected {list(self.shape)}, got {list(shape)} in reshape")
        if not self._layout.is_contiguous():
            raise NotImplementedOp("reshape is not implemented for a non-contiguous view (it never copies)")
        return Tensor(self._storage, Layout(shape, contiguous_strides(shape), self._layout.offset))

    def with_layout(self, shape: Sequence[int], strides: Sequence[int], offset: int) -> "Tensor":
        """An arbitrary strided view of the same storage (checked)."""
        return Tensor.from_storage(self._storage, Layout(tuple(shape), tuple(strides), int(offset)))

    # -- host readback --
    def to_numpy(self) -> np.ndarray:
        """The view's elements in logical order on the host (bf16 as float32)."""
        L = self._layout
        es = self.dtype.size_in_bytes()
        npdt = _np_dtype(self.dtype)
        if numel(L.shape) == 0:
            out = np.zeros(L.shape, dtype=npdt)
        else:
            lo = hi = L.offset
            for d, s in zip(L.shape, L.strides):
                span = (d - 1) * s
                lo, hi = (lo + span, hi) if span < 0 else (lo, hi + span)
            nel = hi - lo + 1
            buf = np.empty(nel, dtype=npdt)
            if self.device.kind == "cpu":
                buf.view(np.uint8)[:] = self._storage._host[lo * es:(hi + 1) * es]
            else:
                check(_lib.lib().oxm_copy(C.c_void_p(buf.ctypes.data), -1,
                                          C.c_void_p(self._storage.ptr + lo * es), self.device.index,
                                          nel * es, _copy_stream(self.device)))
            out = np.lib.stride_tricks.as_strided(buf[L.offset - lo:], shape=L.shape,
                                                  strides=tuple(s * es for s in L.strides)).copy()
        if self.dtype == DType.BF16:
            return bf16_bits_to_f32(out)
        if self.dtype == DType.F16:
            return out.astype(np.float32)
        return out

    def get_f32(self, index: Sequence[int]) -> float:
        """One element as float (tensor.rs:92-99)."""
        off = self._layout.offset_of(index)
        if not self.dtype.is_float():
            raise OxmError(f"get_f32 on a {self.dtype.name} tensor")
        v = Tensor(self._storage, Layout((), (), off)).to_numpy()
        return float(v)

    # -- the C-ABI view --
    def abi_view(self) -> _lib.OxmView:
        L = self._layout
        shape = _lib.i64_array(L.shape)
        strides = _lib.i64_array(L.strides)
        v = _lib.OxmView(C.c_void_p(self._storage.ptr), int(self.dtype), len(L.shape),
                         C.cast(shape, C.POINTER(C.c_int64)), C.cast(strides, C.POINTER(C.c_int64)),
                         int(L.offset), self.device.abi_index)
        v._keep = (shape, strides)  # keep the arrays alive with the struct
        return v

    # -- TensorOps (crates/oxmera-runtime/src/lib.rs:57-72) --
    def matmul(self, rhs: "Tensor") -> "Tensor":
        from .backend import backend_for
        return backend_for(self.device).matmul(self, rhs)

    def sum(self, axes: Sequence[int]) -> "Tensor":
        from .backend import backend_for
        return backend_for(self.device).sum(self, axes)

    def max(self, axes: Sequence[int]) -> "Tensor":
        from .backend import backend_for
        return backend_for(self.device).max(self, axes)

    def _be(self):
        from .backend import backend_for
        return backend_for(self.device)

    def neg(self) -> "Tensor":
        return self._be().neg(self)

    def exp(self) -> "Tensor":
        return self._be().exp(self)

    def ln(self) -> "Tensor":
        return self._be().ln(self)

    def abs(self) -> "Tensor":
        return self._be().abs(self)

    def add(self, rhs: "Tensor") -> "Tensor":
        return self._be().add(self, rhs)

    def sub(self, rhs: "Tensor") -> "Tensor":
        return self._be().sub(self, rhs)

    def mul(self, rhs: "Tensor") -> "Tensor":
        return self._be().mul(self, rhs)

    def div(self, rhs: "Tensor") -> "Tensor":
        return self._be().div(self, rhs)

    def contiguous(self) -> "Tensor":
        """tensor.rs:86-90: fresh contiguous storage; self when already contiguous."""
        return self._be().contiguous(self)

    def __repr__(self) -> str:
        return f"Tensor(shape={list(self.shape)}, strides={list(self._layout.strides)}, " \
               f"offset={self._layout.offset}, dtype={self.dtype.name}, device={self.device})"
