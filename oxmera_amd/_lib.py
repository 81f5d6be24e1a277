"""ctypes binding of the C-ABI in ``include/oxm.h`` (``oxmera_amd/liboxm.so``).

This is the Python twin of the ``oxmera-hip-sys`` FFI crate: it declares
the structs and entry points and maps status codes onto the typed errors of
``oxmera_amd.core``.  Loading fails loudly when the library has not been
built -- there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liboxm.so"

MAX_DIMS = 8

# oxm_status
OK = 0
E_SHAPE_MISMATCH = 1
E_BROADCAST_INCOMPATIBLE = 2
E_DTYPE_MISMATCH = 3
E_UNSUPPORTED_DTYPE = 4
E_DEVICE_MISMATCH = 5
E_INDEX_OUT_OF_BOUNDS = 6
E_RANK_MISMATCH = 7
E_BACKEND_UNAVAILABLE = 8
E_NOT_IMPLEMENTED = 9
E_HIP = 10
E_INVALID_ARGUMENT = 11
E_DIVISION_BY_ZERO = 12

# oxm_act
ACT_NONE = 0
ACT_GELU = 1
ACT_DGELU = 2
ACT_GELU_GRAD = 3  # out = GELU(acc + bias), aux = GELU'(acc + bias)
ACT_MUL_AUX = 4    # out = acc * aux

UN_NEG, UN_EXP, UN_LN, UN_ABS, UN_SIGN = 0, 1, 2, 3, 4
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV, BIN_EQ, BIN_DGELU = 0, 1, 2, 3, 4, 5
RED_SUM, RED_MAX = 0, 1


class OxmView(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("shape", C.POINTER(C.c_int64)),
        ("strides", C.POINTER(C.c_int64)),
        ("offset", C.c_int64),
        ("device", C.c_int32),
    ]


class OxmEpilogue(C.Structure):
    _fields_ = [
        ("bias", C.c_void_p),
        ("bias_dtype", C.c_int32),
        ("act", C.c_int32),
        ("aux", C.c_void_p),
        ("colsum", C.c_void_p),
    ]


# Every entry point of include/oxm.h with its ctypes signature.
_PROTOS = {
    "oxm_version": (C.c_char_p, []),
    "oxm_last_error": (C.c_char_p, []),
    "oxm_backend_name": (C.c_char_p, []),
    "oxm_device_count": (C.c_int, [C.POINTER(C.c_int32)]),
    "oxm_view_byte_range": (C.c_int, [C.POINTER(OxmView), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "oxm_broadcast_shapes": (C.c_int, [C.c_int32, C.POINTER(C.c_int64), C.c_int32, C.POINTER(C.c_int64),
                                       C.POINTER(C.c_int32), C.POINTER(C.c_int64)]),
    "oxm_gemm_infer": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.POINTER(C.c_int32),
                                 C.POINTER(C.c_int64)]),
    "oxm_gemm": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.POINTER(OxmView),
                           C.POINTER(OxmEpilogue), C.c_void_p]),
    "oxm_sum_rows": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_mse_loss_grad": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.POINTER(OxmView),
                                    C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_unary": (C.c_int, [C.c_int32, C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_binary": (C.c_int, [C.c_int32, C.POINTER(OxmView), C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_reduce_infer": (C.c_int, [C.POINTER(OxmView), C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_int32),
                                   C.POINTER(C.c_int64)]),
    "oxm_reduce": (C.c_int, [C.c_int32, C.POINTER(OxmView), C.POINTER(C.c_int32), C.c_int32, C.POINTER(OxmView),
                             C.c_void_p]),
    "oxm_reduce_noalloc": (C.c_int, [C.c_int32, C.POINTER(OxmView), C.POINTER(C.c_int32), C.c_int32,
                                     C.POINTER(OxmView), C.c_void_p]),
    "oxm_copy_view": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_convert": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.c_void_p]),
    "oxm_sgd_step": (C.c_int, [C.POINTER(OxmView), C.POINTER(OxmView), C.POINTER(OxmView), C.c_float, C.c_float,
                               C.c_float, C.c_int32, C.c_void_p]),
    "oxm_alloc": (C.c_int, [C.c_int32, C.c_size_t, C.POINTER(C.c_void_p)]),
    "oxm_free": (C.c_int, [C.c_int32, C.c_void_p]),
    "oxm_copy": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_size_t, C.c_void_p]),
    "oxm_synchronize": (C.c_int, [C.c_int32]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded backend library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 backend first "
                "(python -m oxmera_amd.build); there is no fallback path")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().oxm_last_error().decode()


def exported_symbols() -> list[str]:
    return list(_PROTOS)


def i64_array(values) -> C.Array:
    vals = [int(v) for v in values]
    return (C.c_int64 * max(1, len(vals)))(*vals)
