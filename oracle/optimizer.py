"""Signed gradient descent with linear decay (oracle).

Restates ``mround/reference/optimizer.py:28-158`` and the learning-rate rule of
``mround/schemes.py:307-322``.
"""

from __future__ import annotations

import numpy as np


def resolved_lr(bits: int, iters: int, lr: float | None = None) -> float:
    """``c / iters`` with ``c = 2`` only below 4 bits at >= 1000 steps."""
    if lr is not None:
        return lr
    return (2.0 if (bits < 4 and iters >= 1000) else 1.0) / iters


class LinearDecay:
    """``mround/reference/optimizer.py:28-58``."""

    def __init__(self, initial_lr: float, total_steps: int) -> None:
        if total_steps <= 0:
            raise ValueError(f"total_steps must be positive, got {total_steps}")
        self.initial_lr = initial_lr
        self.total_steps = total_steps

    def __call__(self, step: int) -> float:
        if step >= self.total_steps:
            return 0.0
        return self.initial_lr * (1.0 - step / self.total_steps)


def total_excursion(initial_lr: float, total_steps: int) -> float:
    """``mround/reference/optimizer.py:61-69``."""
    schedule = LinearDecay(initial_lr, total_steps)
    return sum(schedule(step) for step in range(total_steps))


def sign_update(param, grad, lr):
    """``mround/reference/optimizer.py:72-85``."""
    return param - lr * np.sign(grad)


class SignSGD:
    """``mround/reference/optimizer.py:88-158`` (momentum 0 is the method)."""

    def __init__(self, learning_rate, *, momentum: float = 0.0) -> None:
        self.learning_rate = learning_rate
        self.momentum = momentum
        self._step = 0
        self._buffers: dict = {}

    @property
    def step_count(self) -> int:
        return self._step

    def current_lr(self) -> float:
        if isinstance(self.learning_rate, LinearDecay):
            return self.learning_rate(self._step)
        return self.learning_rate

    def apply(self, params: dict, grads: dict) -> dict:
        lr = self.current_lr()
        updated = {}
        for name, value in params.items():
            if name not in grads:
                raise KeyError(f"no gradient supplied for parameter {name!r}")
            grad = grads[name]
            if self.momentum:
                buf = self._buffers.get(name)
                buf = grad.copy() if buf is None else self.momentum * buf + grad
                self._buffers[name] = buf
                grad = buf
            updated[name] = sign_update(value, grad, lr)
        self._step += 1
        return updated
