"""Optimizers over the tape's parameters (the reserved ``oxmera-optim``,
crates/oxmera-optim/src/lib.rs:1-11, defines none yet).

SGD follows torch.optim.SGD with dampening 0, one fused HIP kernel per
parameter (``oxm_sgd_step``): per element in f32, each operation rounded on
its own,

    g = grad (+ weight_decay * p)
    momentum != 0:  v = momentum * v + g;  g = g + momentum * v  (Nesterov)  or  g = v
    p = p - lr * g,  rounded once to p's dtype.

Parameters are F32, BF16 or F16 (updated in place); gradients F32 or the
parameter's dtype; velocity buffers F32, zero before the first step.
"""
from __future__ import annotations

from typing import Iterable, Optional

import numpy as np

from .autograd import Var
from .backend import backend_for
from .core import DType, InvalidArgument
from .tensor import Tensor


class SGD:
    def __init__(self, params: Iterable[Var], lr: float, momentum: float = 0.0, weight_decay: float = 0.0,
                 nesterov: bool = False):
        if not lr > 0 or not np.isfinite(lr):
            raise InvalidArgument(f"SGD: lr must be a positive finite number, got {lr}")
        if momentum < 0 or weight_decay < 0:
            raise InvalidArgument("SGD: momentum and weight_decay must be >= 0")
        if nesterov and momentum == 0:
            raise InvalidArgument("SGD: Nesterov momentum needs momentum > 0")
        self.params = list(params)
        self.lr, self.momentum, self.weight_decay, self.nesterov = lr, momentum, weight_decay, nesterov
        self._velocity: dict = {}

    def _v(self, p: Var) -> Optional[Tensor]:
        if self.momentum == 0:
            return None
        v = self._velocity.get(id(p))
        if v is None:
            v = Tensor.from_numpy(np.zeros(p.t.shape, np.float32), p.t.device, DType.F32)
            self._velocity[id(p)] = v
        return v

    def step(self) -> None:
        """Update every parameter that has a gradient; others are skipped."""
        for p in self.params:
            if p.grad is None:
                continue
            backend_for(p.t.device).sgd_step(p.t, p.grad, self._v(p), self.lr, self.momentum, self.weight_decay,
                                             self.nesterov)

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None
