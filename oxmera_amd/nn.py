"""Layers over the autograd tape (the reserved ``oxmera-nn``,
crates/oxmera-nn/src/lib.rs:1-12): Linear with fused bias/GELU, and the
2-layer MLP of the GEMM backend's training workload."""
from __future__ import annotations

import numpy as np

from . import _lib
from .autograd import Var, linear, mse_loss
from .core import Device, DType
from .tensor import Tensor


class Linear:
    """y = act(x . W + b), W stored [in, out]."""

    def __init__(self, w: Tensor, b: Tensor | None, act: int = _lib.ACT_NONE):
        self.w = Var(w, requires_grad=True)
        self.b = Var(b, requires_grad=True) if b is not None else None
        self.act = act

    @staticmethod
    def init(fan_in: int, fan_out: int, device: Device, dtype: DType, rng: np.random.Generator,
             std: float = 0.02, bias: bool = True, act: int = _lib.ACT_NONE) -> "Linear":
        w = Tensor.from_numpy((rng.standard_normal((fan_in, fan_out), dtype=np.float32) * std), device, dtype)
        b = Tensor.from_numpy((rng.standard_normal((fan_out,), dtype=np.float32) * std), device, dtype) \
            if bias else None
        return Linear(w, b, act)

    def __call__(self, x: Var) -> Var:
        return linear(x, self.w, self.b, self.act)

    def parameters(self) -> list:
        return [self.w] + ([self.b] if self.b is not None else [])

    def zero_grad(self) -> None:
        self.w.grad = None
        if self.b is not None:
            self.b.grad = None


class MLP2:
    """Linear(d -> h) + bias + GELU, Linear(h -> d) + bias."""

    def __init__(self, fc1: Linear, fc2: Linear):
        self.fc1, self.fc2 = fc1, fc2

    def __call__(self, x: Var) -> Var:
        return self.fc2(self.fc1(x))

    def parameters(self) -> list:
        return self.fc1.parameters() + self.fc2.parameters()

    def train_step(self, x: Var, target: Tensor) -> Var:
        """Forward, MSE against ``target`` and backward; returns the loss."""
        self.fc1.zero_grad()
        self.fc2.zero_grad()
        x.grad = None
        loss = mse_loss(self(x), target)
        loss.backward()
        return loss
