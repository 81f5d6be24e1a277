"""ctypes wrapper of the CPU oracle (``oracle/oxm_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg, always as the checker, never by the
product package ``oxmera_amd``.

The oracle restates oxmera's reference matmul (CpuBackend::matmul,
crates/oxmera-cpu/src/lib.rs:71-76, specified by
exercises/a4-reference-matmul/tests/spec.rs) as three naive loops reading
through element strides with f32 ascending-k accumulation, extended with
batch broadcasting, bf16/f16 widening and the fused epilogue.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboxm_oracle.so"

F32, F64, BF16, F16 = 0, 1, 6, 7
ACT_NONE, ACT_GELU, ACT_DGELU, ACT_GELU_GRAD, ACT_MUL_AUX = 0, 1, 2, 3, 4
STATUS = {0: "ok", 1: "ShapeMismatch", 2: "BroadcastIncompatible", 3: "DTypeMismatch", 4: "UnsupportedDType",
          7: "RankMismatch"}


class _View(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.POINTER(C.c_int64)), ("strides", C.POINTER(C.c_int64)),
                ("offset", C.c_int64), ("device", C.c_int32)]


def build() -> Path:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        L.oxm_oracle_gemm.restype = C.c_int
        L.oxm_oracle_gemm.argtypes = [C.POINTER(_View), C.POINTER(_View), C.c_int, C.c_void_p, C.c_int, C.c_int,
                                      C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_int]
        L.oxm_oracle_broadcast.restype = C.c_int
        L.oxm_oracle_broadcast.argtypes = [C.c_int, C.POINTER(C.c_int64), C.c_int, C.POINTER(C.c_int64),
                                           C.POINTER(C.c_int), C.POINTER(C.c_int64)]
        for n in ("oxm_oracle_gelu", "oxm_oracle_dgelu"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [C.c_float]
        L.oxm_oracle_colsum.restype = None
        L.oxm_oracle_colsum.argtypes = [C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p]
        _lib = L
    return _lib


class OracleError(Exception):
    def __init__(self, code: int):
        super().__init__(STATUS.get(code, str(code)))
        self.code = code
        self.kind = STATUS.get(code, str(code))


class StridedView:
    """A strided view of a flat host buffer: the oracle's operand."""

    def __init__(self, buf: np.ndarray, dtype: int, shape, strides, offset: int = 0):
        self.buf = np.ascontiguousarray(buf)
        self.dtype = dtype
        self.shape = tuple(int(s) for s in shape)
        self.strides = tuple(int(s) for s in strides)
        self.offset = int(offset)

    @staticmethod
    def contiguous(arr: np.ndarray, dtype: int | None = None) -> "StridedView":
        arr = np.ascontiguousarray(arr)
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.float64): F64, np.dtype(np.float16): F16}[arr.dtype]
        strides = [0] * arr.ndim
        acc = 1
        for i in range(arr.ndim - 1, -1, -1):
            strides[i] = acc
            acc *= arr.shape[i]
        return StridedView(arr.reshape(-1), dtype, arr.shape, strides, 0)

    def permute(self, perm) -> "StridedView":
        return StridedView(self.buf, self.dtype, [self.shape[p] for p in perm], [self.strides[p] for p in perm],
                           self.offset)

    def _struct(self):
        shp = (C.c_int64 * max(1, len(self.shape)))(*self.shape)
        std = (C.c_int64 * max(1, len(self.strides)))(*self.strides)
        v = _View(self.buf.ctypes.data, self.dtype, len(self.shape), C.cast(shp, C.POINTER(C.c_int64)),
                  C.cast(std, C.POINTER(C.c_int64)), self.offset, -1)
        return v, (shp, std)


def out_shape(a: StridedView, b: StridedView) -> tuple:
    na, nb = a.shape[:-2], b.shape[:-2]
    sa = (C.c_int64 * max(1, len(na)))(*na)
    sb = (C.c_int64 * max(1, len(nb)))(*nb)
    n = C.c_int(0)
    o = (C.c_int64 * 8)()
    st = lib().oxm_oracle_broadcast(len(na), sa, len(nb), sb, C.byref(n), o)
    if st:
        raise OracleError(st)
    return tuple(o[i] for i in range(n.value)) + (a.shape[-2], b.shape[-1])


def matmul(a: StridedView, b: StridedView, *, out_dtype: int = F32, bias: np.ndarray | None = None,
           bias_dtype: int = F32, act: int = ACT_NONE, aux: np.ndarray | None = None,
           rows: np.ndarray | None = None, want_aux: bool = False, nthreads: int | None = None):
    """The reference matmul.  Returns C (f32 array, or uint16 bits for a
    16-bit out_dtype).  ``rows``: flattened (batch*M + m) rows to compute;
    the result is then [len(rows), N].  With ``want_aux`` (GELU / GELU_GRAD),
    returns (C, aux): the pre-activation, or GELU' of it."""
    if len(a.shape) < 2 or len(b.shape) < 2:
        raise OracleError(7)
    shape = out_shape(a, b) if a.shape[-1] == b.shape[-2] else None
    if shape is None:
        raise OracleError(1)
    N = shape[-1]
    npdt = np.float32 if out_dtype == F32 else (np.float64 if out_dtype == F64 else np.uint16)
    if rows is not None:
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        oshape = (len(rows), N)
    else:
        oshape = shape
    out = np.zeros(oshape, dtype=npdt)
    aux_out = np.zeros(oshape, dtype=npdt) if want_aux else None
    va, ka = a._struct()
    vb, kb = b._struct()
    bias_c = np.ascontiguousarray(bias) if bias is not None else None
    aux_c = np.ascontiguousarray(aux) if aux is not None else None
    # the GPU box gives one process a 16-core share whatever cpu_count() reports
    nt = nthreads or min(os.cpu_count() or 1, 16)
    st = lib().oxm_oracle_gemm(C.byref(va), C.byref(vb), out_dtype,
                               bias_c.ctypes.data if bias_c is not None else None, bias_dtype, act,
                               aux_c.ctypes.data if aux_c is not None else None,
                               rows.ctypes.data if rows is not None else None,
                               len(rows) if rows is not None else 0, out.ctypes.data,
                               aux_out.ctypes.data if aux_out is not None else None, nt)
    if st:
        raise OracleError(st)
    return (out, aux_out) if want_aux else out


def gelu(x: float) -> float:
    return lib().oxm_oracle_gelu(x)


def dgelu(x: float) -> float:
    return lib().oxm_oracle_dgelu(x)


def colsum(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    R, Cc = x.shape
    out = np.zeros(Cc, dtype=np.float32)
    lib().oxm_oracle_colsum(x.ctypes.data, dtype, R, Cc, out.ctypes.data)
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (same rule as the oracle's C)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
