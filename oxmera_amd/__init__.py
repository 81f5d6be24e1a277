"""oxmera_amd -- the MI355X (gfx950) GEMM backend for oxmera.

Layers:
  ``liboxm.so``   C-ABI (include/oxm.h): HIP MFMA GEMM kernels for strided
                  views, fused bias/GELU epilogues, bias-gradient and MSE kernels,
                  elementwise / reduction / copy kernels, the fused SGD update.
  ``core``        oxmera-core vocabulary (DType, Layout, Device, typed errors).
  ``tensor``      Storage / Tensor views (never copied on the GEMM path).
  ``backend``     HipBackend (Matmul, Unary, Binary, Reduce ops) and the device registry.
  ``autograd``/``nn``/``optim``  the tape, Linear layers and SGD.
"""
from . import _lib
from .core import (BackendUnavailable, BroadcastIncompatible, Device, DeviceMismatch, DivisionByZero, DType,
                   DTypeMismatch, HipError, IndexOutOfBounds, InvalidArgument, Layout, NotImplementedOp, OxmError, RankMismatch,
                   ShapeMismatch, UnsupportedDType, broadcast_shapes, contiguous_strides, numel)
from .tensor import Storage, Tensor, bf16_bits_to_f32, f32_to_bf16_bits
from .backend import HipBackend, backend_for, device_count, init, register_backend

ACT_NONE, ACT_GELU, ACT_DGELU = _lib.ACT_NONE, _lib.ACT_GELU, _lib.ACT_DGELU
ACT_GELU_GRAD, ACT_MUL_AUX = _lib.ACT_GELU_GRAD, _lib.ACT_MUL_AUX

__all__ = [
    "BackendUnavailable", "BroadcastIncompatible", "Device", "DeviceMismatch", "DivisionByZero", "DType",
    "DTypeMismatch",
    "HipError", "IndexOutOfBounds", "InvalidArgument", "Layout", "NotImplementedOp", "OxmError", "RankMismatch",
    "ShapeMismatch", "UnsupportedDType", "broadcast_shapes", "contiguous_strides", "numel", "Storage", "Tensor",
    "bf16_bits_to_f32", "f32_to_bf16_bits", "HipBackend", "backend_for", "device_count", "init",
    "register_backend", "ACT_NONE", "ACT_GELU", "ACT_DGELU", "ACT_GELU_GRAD", "ACT_MUL_AUX",
]
