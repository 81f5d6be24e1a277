"""oxmera-core vocabulary, mirrored for the HIP backend's host side.

Mirrors ``crates/oxmera-core/src``:
  - ``DType``                     dtype.rs:9-34 (+ BF16, F16 carried end to end here)
  - ``Shape`` helpers, ``numel``  shape.rs:11-34
  - ``broadcast_shapes``          shape.rs:45-58 (computed by the C++ host layer)
  - ``Strides``/``Layout``        layout.rs:6-62
  - ``Device``                    device.rs:10-31 (+ a ROCm variant)
  - ``Error`` taxonomy            error.rs:14-105
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Sequence

from . import _lib

# ---- dtypes -----------------------------------------------------------------


class DType(enum.IntEnum):
    """Element type; values equal the C-ABI's ``oxm_dtype``."""
    F32 = 0
    F64 = 1
    I32 = 2
    I64 = 3
    U8 = 4
    Bool = 5
    BF16 = 6
    F16 = 7

    def size_in_bytes(self) -> int:
        return {0: 4, 1: 8, 2: 4, 3: 8, 4: 1, 5: 1, 6: 2, 7: 2}[int(self)]

    def is_float(self) -> bool:
        return self in (DType.F32, DType.F64, DType.BF16, DType.F16)


# ---- devices ------------------------------------------------------------------


@dataclass(frozen=True)
class Device:
    """Where storage lives: ``Device.cpu()`` or ``Device.rocm(i)``."""
    kind: str
    index: int = 0

    @staticmethod
    def cpu() -> "Device":
        return Device("cpu", 0)

    @staticmethod
    def rocm(index: int = 0) -> "Device":
        return Device("rocm", index)

    def kind_name(self) -> str:
        return self.kind

    @property
    def abi_index(self) -> int:
        """-1 for host memory, else the HIP device index (oxm_view.device)."""
        return -1 if self.kind == "cpu" else self.index

    def __repr__(self) -> str:
        return "Cpu" if self.kind == "cpu" else f"Rocm {{ index: {self.index} }}"


# ---- errors -------------------------------------------------------------------


class OxmError(Exception):
    """Base of the typed errors (``oxmera_core::Error``)."""
    code = -1


class ShapeMismatch(OxmError):
    code = _lib.E_SHAPE_MISMATCH


class BroadcastIncompatible(OxmError):
    code = _lib.E_BROADCAST_INCOMPATIBLE

    def __init__(self, msg: str, lhs=None, rhs=None):
        super().__init__(msg)
        self.lhs, self.rhs = lhs, rhs


class DTypeMismatch(OxmError):
    code = _lib.E_DTYPE_MISMATCH


class UnsupportedDType(OxmError):
    code = _lib.E_UNSUPPORTED_DTYPE


class DeviceMismatch(OxmError):
    code = _lib.E_DEVICE_MISMATCH


class IndexOutOfBounds(OxmError):
    code = _lib.E_INDEX_OUT_OF_BOUNDS

    def __init__(self, msg: str, index=None, shape=None):
        super().__init__(msg)
        self.index, self.shape = index, shape


class RankMismatch(OxmError):
    code = _lib.E_RANK_MISMATCH

    def __init__(self, msg: str, index_rank=None, shape_rank=None):
        super().__init__(msg)
        self.index_rank, self.shape_rank = index_rank, shape_rank


class BackendUnavailable(OxmError):
    code = _lib.E_BACKEND_UNAVAILABLE


class NotImplementedOp(OxmError):
    code = _lib.E_NOT_IMPLEMENTED


class HipError(OxmError):
    code = _lib.E_HIP


class InvalidArgument(OxmError):
    code = _lib.E_INVALID_ARGUMENT


class DivisionByZero(OxmError):
    """Integer division by zero: the typed error BinaryOps::div promises
    (crates/oxmera-ops/src/lib.rs:47-48)."""
    code = _lib.E_DIVISION_BY_ZERO


_BY_CODE = {cls.code: cls for cls in (ShapeMismatch, BroadcastIncompatible, DTypeMismatch, UnsupportedDType,
                                      DeviceMismatch, IndexOutOfBounds, RankMismatch, BackendUnavailable,
                                      NotImplementedOp, HipError, InvalidArgument, DivisionByZero)}


def check(status: int) -> None:
    """Raise the typed error for a non-OK C-ABI status."""
    if status != _lib.OK:
        raise _BY_CODE.get(status, OxmError)(_lib.last_error())


# ---- shapes, strides, layouts -----------------------------------------------


def numel(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def contiguous_strides(shape: Sequence[int]) -> tuple[int, ...]:
    """Row-major element strides (layout.rs:58-62)."""
    out = [0] * len(shape)
    acc = 1
    for i in range(len(shape) - 1, -1, -1):
        out[i] = acc
        acc *= int(shape[i])
    return tuple(out)


def broadcast_shapes(lhs: Sequence[int], rhs: Sequence[int]) -> tuple[int, ...]:
    """NumPy broadcasting (shape.rs:45-58), computed by the C++ host layer."""
    a, b = _lib.i64_array(lhs), _lib.i64_array(rhs)
    nout = C.c_int32(0)
    out = (C.c_int64 * _lib.MAX_DIMS)()
    st = _lib.lib().oxm_broadcast_shapes(len(lhs), a, len(rhs), b, C.byref(nout), out)
    if st == _lib.E_BROADCAST_INCOMPATIBLE:
        raise BroadcastIncompatible(_lib.last_error(), tuple(lhs), tuple(rhs))
    check(st)
    return tuple(out[i] for i in range(nout.value))


@dataclass(frozen=True)
class Layout:
    """Shape, signed element strides and element offset (layout.rs:24-34)."""
    shape: tuple[int, ...]
    strides: tuple[int, ...]
    offset: int = 0

    @staticmethod
    def contiguous(shape: Sequence[int]) -> "Layout":
        shape = tuple(int(d) for d in shape)
        return Layout(shape, contiguous_strides(shape), 0)

    def offset_of(self, index: Sequence[int]) -> int:
        """Storage offset of a logical index (layout.rs:43-49)."""
        if len(index) != len(self.shape):
            raise RankMismatch(f"rank mismatch: index of rank {len(index)} against shape of rank {len(self.shape)}",
                               len(index), len(self.shape))
        for i, d in zip(index, self.shape):
            if not 0 <= i < d:
                raise IndexOutOfBounds(f"index {list(index)} out of bounds for shape {list(self.shape)}",
                                       list(index), tuple(self.shape))
        return self.offset + sum(i * s for i, s in zip(index, self.strides))

    def is_contiguous(self) -> bool:
        """Row-major contiguity; scalars and empty tensors count (layout.rs:51-55)."""
        if numel(self.shape) == 0:
            return True
        expect = 1
        for d, s in zip(reversed(self.shape), reversed(self.strides)):
            if d != 1 and s != expect:
                return False
            expect *= d
        return True
